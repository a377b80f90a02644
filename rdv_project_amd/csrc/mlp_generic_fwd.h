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
//
// This header holds the kernel and its launch templates; mlp_generic.hip
// dispatches, and the 8-tile instantiations (the largest to compile) live in
// mlp_generic8.hip and mlp_generic8g.hip so that the sources build in parallel.
#ifndef RDV_MLP_GENERIC_FWD_H
#define RDV_MLP_GENERIC_FWD_H

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

// Layer-0 K chunks held in registers ahead of their tile (PRE kernels).
constexpr int kGenPreChunks = 4;

// PRE: raw 16-byte aligned input of at most kGenPreChunks K chunks (D <= 64).
// Each wave claims its next tile when it starts one, and loads that tile's
// input rows into registers as soon as the current tile's layer-0 MFMAs are
// issued, so the loads are in flight during the hidden layers instead of being
// waited for chunk by chunk.  Otherwise layer 0 loads each chunk when it needs it.
template <int MT, bool LDSW, bool PRE>
__global__ __launch_bounds__(64 * gen_waves<MT>(), 1) void mlp_generic_f16_kernel(GenFwdArgs a) {
  constexpr int kGenWaves = gen_waves<MT>();
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int s_next;
  const GenNet& g = a.net;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int h0 = lane >> 5, col = lane & 31;
  const bool has_bias = packed_has_bias(a.packed);

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

  // PRE: this lane's 16-byte pieces of K chunks 0 .. 3 (features 16 c + 8 h0 +
  // 4 q + 0..3 in raw[2 c + q]) of a tile's row; pieces past D are loaded from
  // column 0 (in bounds) and replaced by zeros when converted into xb, the
  // tile's layer-0 B fragments, at the start of the tile.  (Converting at the
  // end of the previous tile instead, before its output stores, measured 5%
  // slower.)
  f32x4 raw[2 * kGenPreChunks];
  half8 xb[kGenPreChunks];
  auto load_raw = [&](int tile) {
    const int64_t r = (t_begin + tile) * 32 + col;
    const float* xp = a.x + (r < a.nrows ? r : a.nrows - 1) * D;
#pragma unroll
    for (int i = 0; i < 2 * kGenPreChunks; ++i) {
      const int f = 16 * (i >> 1) + 8 * h0 + 4 * (i & 1);
      raw[i] = *reinterpret_cast<const f32x4*>(xp + (f < D ? f : 0));
    }
  };
  auto convert_raw = [&]() {
    const f32x4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < kGenPreChunks; ++c) {
      const int f = 16 * c + 8 * h0;
      const f32x4 v0 = f < D ? raw[2 * c] : zero4;
      const f32x4 v1 = f + 4 < D ? raw[2 * c + 1] : zero4;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xb[c][j] = half_t(v0[j]);
        xb[c][4 + j] = half_t(v1[j]);
      }
    }
  };
  if constexpr (PRE) {
    if (nt > 0) {
      load_raw(wave < nt ? wave : nt - 1);
    }
  }

  for (int t = wave; t < nt;) {
    const int tn = claim();
    if constexpr (PRE) convert_raw();
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
    auto after0 = [&]() {
      if constexpr (PRE) load_raw(tn < nt ? tn : nt - 1);
    };
    auto l0 = [&](int c) -> half8 {
      if constexpr (PRE) return xb[c];
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
                // a cached store: the two lane halves write alternate 16-byte pieces of each
                // row, and the L2 merges them into whole lines (non-temporal stores left
                // half lines: 1.40x the output bytes)
                *reinterpret_cast<f32x4*>(yr + r0) = v;
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
    gen_chain<MT, PRE ? kGenPreChunks : 0>(g, cx, wf, l0, sink, after0);
    t = tn;
  }
}

template <int MT, bool LDSW, bool PRE>
static int launch_generic_pre(const GenFwdArgs& a, int64_t blocks, size_t lds, hipStream_t stream) {
  static bool attr = false;
  if (LDSW && !attr) {
    RDV_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&mlp_generic_f16_kernel<MT, LDSW, PRE>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, int(kGenLdsCap)));
    attr = true;
  }
  mlp_generic_f16_kernel<MT, LDSW, PRE><<<dim3(unsigned(blocks)), dim3(64 * gen_waves<MT>()), lds, stream>>>(a);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

// The register prefetch of layer 0's input (PRE) serves raw 16-byte aligned
// inputs of at most kGenPreChunks chunks with the weights in LDS; the 8-tile
// chains, at one wave per SIMD with their accumulators in AGPRs, and the
// global-weight kernels, whose addresses take more registers, have none to
// spare for it.
template <int MT, bool LDSW>
static int launch_generic_t(const GenFwdArgs& a, int64_t blocks, size_t lds, hipStream_t stream) {
  if constexpr (MT <= 4 && LDSW) {
    if (a.vec_in && a.net.kc[0] <= kGenPreChunks) return launch_generic_pre<MT, LDSW, true>(a, blocks, lds, stream);
  }
  return launch_generic_pre<MT, LDSW, false>(a, blocks, lds, stream);
}

// The 8-tile kernels (weights in LDS / in global memory), each in its own source.
int launch_generic_mt8_lds(const GenFwdArgs& a, int64_t blocks, size_t lds, hipStream_t stream);
int launch_generic_mt8_global(const GenFwdArgs& a, int64_t blocks, hipStream_t stream);

}  // namespace rdv

#endif  // RDV_MLP_GENERIC_FWD_H
