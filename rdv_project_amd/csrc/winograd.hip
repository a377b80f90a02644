// Winograd F(2x2, 3x3) convolution on the fp16 matrix cores.
//
// Replaces Conv2DTensorOpWinograd3x3 (src/rdv/domain/nn.py:1002-1087,
// src/rdv/shaders/tensors/conv2d_tensor_op_winograd3x3.h:95-178) with the same
// numerics: U = G g G^T in fp32 rounded to fp16 (nn.py:522-538); per tile and
// input channel V = B^T d B in fp32 rounded to fp16 (.h:59-78, 136; the
// pipelined kernel's matrix-core sum of the same four terms, below); 16
// channel-reduction GEMMs with fp32 accumulation (.h:142-161); Y = A^T M A in
// fp32 plus the fp32 bias (.h:80-93, 169-173); optional ReLU epilogue.
//
// MI355X mapping (v_mfma_f32_16x16x32_f16: A 16x32, B 32x16, D 16x16):
//   M = 16 output channels (one wave per 16-channel group), N = 16 Winograd
//   tiles, K = 32 input channels.  Lane l holds
//     A: U[p][ci = 32 kc + 8 (l/16) + j][co = 16 g + l%16]          (VGPRs, packed)
//     B: V[p][tile l%16][ci = 32 kc + 8 (l/16) + j]                 (LDS, ds_read_b128)
//     D: M[p][co = 16 g + 4 (l/16) + j][tile l%16], j = 0..3
//   so every lane holds all 16 domain positions of its (tile, 4 channels) and
//   the inverse transform runs in registers: for each row a of the 4x4 domain,
//   the four M[a][b] are reduced over b and folded into the 2x2 output.
//   The reference's structure (one lane per tile re-reading its 4x4xCIN patch
//   from global memory for every (position, channel block) pair, .h:113-137) is
//   replaced by one staging of the haloed input in LDS per tile group.
//
// Work decomposition (generic kernel, any layout and dtype): a tile group is 16
// consecutive tiles of one tile row (2 output rows x 32 output columns).  Each
// block owns a contiguous range of groups; per group it stages the 4 x 34 x CIN
// input region in LDS (fp32), transforms it to V in B-fragment order (fp16),
// then every wave evaluates its 16 output channels for the 16 tiles.  NCHW fp16
// input takes winograd3x3_pipe_kernel (below): the same transforms and GEMMs,
// input rows by DMA, and the input transform of one tile row overlapped with
// the GEMMs of the previous one.
#include <algorithm>
#include <type_traits>

#include "rdv_common.h"

namespace rdv {

constexpr int kWgTiles = 16;               // tiles per group (MFMA N)
constexpr int kWgCols = 2 * kWgTiles + 2;  // staged input columns (34)

// ---------------------------------------------------------------- weights
// U for (p, ci, co) following nn.py:532-538: T = G g (3 terms per element),
// then U = T G^T (3 terms), in fp32, rounded to fp16.  g[r][s] = w(ci, co, r, s).
__device__ __forceinline__ float winograd_u(const float g[3][3], int a, int b) {
  const float G[4][3] = {{1.0f, 0.0f, 0.0f}, {0.5f, 0.5f, 0.5f}, {0.5f, -0.5f, 0.5f}, {0.0f, 0.0f, 1.0f}};
  float t[3];
#pragma unroll
  for (int s = 0; s < 3; ++s) t[s] = G[a][0] * g[0][s] + G[a][1] * g[1][s] + G[a][2] * g[2][s];
  return t[0] * G[b][0] + t[1] * G[b][1] + t[2] * G[b][2];
}

// One thread per packed element: Upk[p][kc][g][lane][j] (fp16), zero for padded channels.
__global__ void winograd_transform_weight_kernel(const void* __restrict__ w, int w_layout, int w_dtype, int cin,
                                                 int cout, int kc_n, int g_n, half_t* __restrict__ U) {
  const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = int64_t(16) * kc_n * g_n * 64 * 8;
  if (e >= total) return;
  const int j = int(e & 7);
  const int lane = int((e >> 3) & 63);
  int64_t r = e >> 9;
  const int g = int(r % g_n);
  r /= g_n;
  const int kc = int(r % kc_n);
  const int p = int(r / kc_n);
  const int ci = 32 * kc + 8 * (lane >> 4) + j;
  const int co = 16 * g + (lane & 15);
  float v = 0.0f;
  if (ci < cin && co < cout) {
    float gm[3][3];
#pragma unroll
    for (int rr = 0; rr < 3; ++rr)
#pragma unroll
      for (int ss = 0; ss < 3; ++ss) {
        // reference layout [3][3][CIN][COUT]; KCRS = PyTorch OIHW [COUT][CIN][3][3]
        const int64_t idx = w_layout == RDV_WLAYOUT_RSCK ? ((int64_t(rr) * 3 + ss) * cin + ci) * cout + co
                                                         : ((int64_t(co) * cin + ci) * 3 + rr) * 3 + ss;
        gm[rr][ss] = w_dtype == RDV_DTYPE_F16 ? float(reinterpret_cast<const half_t*>(w)[idx])
                                              : reinterpret_cast<const float*>(w)[idx];
      }
    v = winograd_u(gm, p >> 2, p & 3);
  }
  // Round to fp32 first, as the reference does: without this barrier the
  // compiler fuses the last fma with the fp16 conversion (v_fma_mix, one
  // rounding), which differs from fp32-then-fp16 on exact fp16 ties.
  asm volatile("" : "+v"(v));
  U[e] = half_t(v);
}

// ---------------------------------------------------------------- forward
struct WinogradArgs {
  const void* x;
  const half_t* U;
  const float* bias;  // may be null
  void* y;
  int batch, H, W, cin, cout;
  int in_layout, in_dtype, out_layout, out_dtype;
  int relu;
  int th, seg;        // tile rows per image, 16-tile segments per tile row
  int64_t ngroups;    // batch * th * seg
  int rows_per_item;  // pipelined kernel: tile rows per work item
  int chunks;         // pipelined kernel: work items per strip (ceil(th / rows_per_item))
  int64_t items;      // pipelined kernel: batch * seg * chunks
};

// The 16 channel-reduction GEMMs of one 16-tile group for this wave's 16
// output channels (A = U from registers, B = V fragments from LDS), the
// inverse transform folded column by column in the reference's order
// (_winograd_inv, .h:80-93):
//   t0[b] = (M[0][b] + M[1][b]) + M[2][b],  t1[b] = (M[1][b] - M[2][b]) - M[3][b]
//   Y[i][0] = (t_i[0] + t_i[1]) + t_i[2],   Y[i][1] = (t_i[1] - t_i[2]) - t_i[3]
// then + bias, optional ReLU, and the store of the 2x2 outputs of tile
// lane % 16 for channels 16 g + 4 (lane / 16) + 0..3 (`bias` holds those
// four channels' biases).
template <int KC>
__device__ __forceinline__ void wg_gemm(const half8 (&u)[16][KC], const half8* sv, int lane, f32x4 (&yv)[2][2]) {
  f32x4 y00, y01, y10, y11;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    f32x4 ma[4];
#pragma unroll
    for (int ra = 0; ra < 4; ++ra) {
      const int p = 4 * ra + b;
      f32x4 acc = {};
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(u[p][kc], sv[(p * KC + kc) * 64 + lane], acc, 0, 0, 0);
      ma[ra] = acc;
    }
    const f32x4 t0 = ma[0] + ma[1] + ma[2];
    const f32x4 t1 = ma[1] - ma[2] - ma[3];
    if (b == 0) {
      y00 = t0;
      y10 = t1;
    } else if (b == 1) {
      y00 += t0;
      y01 = t0;
      y10 += t1;
      y11 = t1;
    } else if (b == 2) {
      y00 += t0;
      y01 -= t0;
      y10 += t1;
      y11 -= t1;
    } else {
      y01 -= t0;
      y11 -= t1;
    }
  }
  yv[0][0] = y00;
  yv[0][1] = y01;
  yv[1][0] = y10;
  yv[1][1] = y11;
}

template <int KC>
__device__ __forceinline__ void wg_gemm_store(const half8 (&u)[16][KC], const half8* sv, int lane, int g,
                                              const f32x4& bias, const WinogradArgs& a, int img, int tr, int seg) {
  f32x4 yv[2][2];
  wg_gemm(u, sv, lane, yv);
  const int hw = a.H * a.W;
  const int n = lane & 15;
  const int tc = seg * kWgTiles + n;
  const int co0 = 16 * g + 4 * (lane >> 4);
  if (tc >= a.W / 2 || co0 >= a.cout) return;
  const int oh = 2 * tr, ow = 2 * tc;
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const float bb = bias[jj];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        float val = yv[i][j][jj] + bb;
        if (a.relu) val = fmaxf(val, 0.0f);
        yv[i][j][jj] = val;
      }
  }
  if (a.out_layout == RDV_LAYOUT_CHW) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int64_t o = (int64_t(img) * a.cout + co0 + jj) * hw + int64_t(oh + i) * a.W + ow;
        if (a.out_dtype == RDV_DTYPE_F16) {
          half2v hv = {half_t(yv[i][0][jj]), half_t(yv[i][1][jj])};
          __builtin_nontemporal_store(hv, reinterpret_cast<half2v*>(static_cast<half_t*>(a.y) + o));
        } else {
          f32x2 fv = {yv[i][0][jj], yv[i][1][jj]};
          __builtin_nontemporal_store(fv, reinterpret_cast<f32x2*>(static_cast<float*>(a.y) + o));
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int64_t o = (int64_t(img) * hw + int64_t(oh + i) * a.W + ow + j) * a.cout + co0;
        if (a.out_dtype == RDV_DTYPE_F16) {
          half4 hv = {half_t(yv[i][j][0]), half_t(yv[i][j][1]), half_t(yv[i][j][2]), half_t(yv[i][j][3])};
          __builtin_nontemporal_store(hv, reinterpret_cast<half4*>(static_cast<half_t*>(a.y) + o));
        } else {
          __builtin_nontemporal_store(yv[i][j], reinterpret_cast<f32x4*>(static_cast<float*>(a.y) + o));
        }
      }
  }
}

// 16 zero bytes: the source of every load that falls outside the operands.
__device__ __attribute__((aligned(16))) uint32_t g_wg_zero16[4] = {0u, 0u, 0u, 0u};

// The four biases of this lane's output channels 16 g + 4 (lane / 16) + 0..3
// (zero past cout or without a bias).  The loads are unconditional (clamped
// index, the zero block for a null bias), so no wait is forced on loads issued
// before them.
__device__ __forceinline__ f32x4 wg_lane_bias(const WinogradArgs& a, int g, int lane) {
  const int co0 = 16 * g + 4 * (lane >> 4);
  const float* src = a.bias ? a.bias : reinterpret_cast<const float*>(g_wg_zero16);
  const int last = a.bias ? a.cout - 1 : 0;
  f32x4 b;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = co0 + j;
    const float v = src[c < last ? c : last];
    b[j] = c < a.cout ? v : 0.0f;
  }
  return b;
}

// Block: 4 waves; wave w owns output channels 16 (4 blockIdx.y + w) + 0..15
// (waves past COUT only help with staging).  IN_F16 / IN_CHW select the input
// element type and layout at compile time.
template <int KC, bool IN_F16, bool IN_CHW>
__global__ __launch_bounds__(256, 2) void winograd3x3_kernel(WinogradArgs a) {
  using in_t = typename std::conditional<IN_F16, half_t, float>::type;
  constexpr int CINP = 32 * KC;                          // padded input channels
  constexpr int XS = CINP + 4;                           // LDS pixel stride (floats): 8-byte aligned, fewer bank conflicts
  constexpr int kRegion = 4 * kWgCols * CINP;            // staged elements per group
  constexpr int kPer = (kRegion + 255) / 256;            // per thread
  __shared__ float sin_[4 * kWgCols * XS];
  __shared__ half8 sv[16 * KC * 64];                     // V fragments [p][kc][lane]
  const int lane = threadIdx.x & 63;
  const int g = blockIdx.y * 4 + (threadIdx.x >> 6);     // output channel group (16 channels)
  const bool active = 16 * g < a.cout;
  const int hw = a.H * a.W;
  const in_t* __restrict__ x = static_cast<const in_t*>(a.x);

  // this wave's U fragments, resident for the whole block
  half8 u[16][KC];
  const int g_n = (a.cout + 15) / 16;
  const int gu = active ? g : 0;
#pragma unroll
  for (int p = 0; p < 16; ++p)
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
      u[p][kc] = reinterpret_cast<const half8*>(a.U)[((int64_t(p) * KC + kc) * g_n + gu) * 64 + lane];

  const f32x4 bias = wg_lane_bias(a, gu, lane);
  const int64_t per_block = (a.ngroups + gridDim.x - 1) / gridDim.x;
  const int64_t g_begin = int64_t(blockIdx.x) * per_block;
  const int64_t g_end = g_begin + per_block < a.ngroups ? g_begin + per_block : a.ngroups;

  // Loads of group grp's 4 x 34 x CINP input region into registers: every load
  // is unconditional (clamped offset from the image's base) so that all are in
  // flight at once; the zero padding is applied by a select.
  auto load_region = [&](int64_t grp, float (&v)[kPer]) {
    const int seg = int(grp % a.seg);
    const int64_t rest = grp / a.seg;
    const int tr = int(rest % a.th);
    const int img = int(rest / a.th);
    const int ih0 = 2 * tr - 1, iw0 = 2 * (seg * kWgTiles) - 1;
    const in_t* __restrict__ base = x + int64_t(img) * a.cin * hw;
    // opaque copy of the thread index: keeps the compiler from hoisting kPer
    // per-element index decompositions out of the group loop into registers
    int tid = int(threadIdx.x);
    asm volatile("" : "+v"(tid));
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = k * 256 + tid;
      int ci, c, r;
      if constexpr (IN_CHW) {  // consecutive threads walk a row segment of one channel
        c = i % kWgCols;
        r = (i / kWgCols) % 4;
        ci = i / (4 * kWgCols);
      } else {                 // consecutive threads walk the channels of one pixel
        ci = i % CINP;
        c = (i / CINP) % kWgCols;
        r = i / (CINP * kWgCols);
      }
      const int ih = ih0 + r, iw = iw0 + c;
      const bool ok = i < kRegion && ci < a.cin && ih >= 0 && ih < a.H && iw >= 0 && iw < a.W;
      int off = IN_CHW ? ci * hw + ih * a.W + iw : (ih * a.W + iw) * a.cin + ci;
      off = ok ? off : 0;
      const float val = float(base[off]);
      v[k] = ok ? val : 0.0f;
    }
  };
  auto park_region = [&](const float (&v)[kPer]) {
    int tid = int(threadIdx.x);
    asm volatile("" : "+v"(tid));
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = k * 256 + tid;
      if (i < kRegion) {
        int ci, c, r;
        if constexpr (IN_CHW) {
          c = i % kWgCols;
          r = (i / kWgCols) % 4;
          ci = i / (4 * kWgCols);
        } else {
          ci = i % CINP;
          c = (i / CINP) % kWgCols;
          r = i / (CINP * kWgCols);
        }
        sin_[(r * kWgCols + c) * XS + ci] = v[k];
      }
    }
  };

  if (g_begin < g_end) {
    float v[kPer];
    load_region(g_begin, v);
    park_region(v);
  }
  __syncthreads();

  for (int64_t grp = g_begin; grp < g_end; ++grp) {
    const int seg = int(grp % a.seg);
    const int64_t rest = grp / a.seg;
    const int tr = int(rest % a.th);
    const int img = int(rest / a.th);

    // ---- V = B^T d B per (tile, 2 channels), fp32 -> fp16, B-fragment order
    for (int unit = threadIdx.x; unit < kWgTiles * (CINP / 2); unit += 256) {
      const int n = unit % kWgTiles;
      const int q = unit / kWgTiles;  // channel pair
      // rows first, exactly as _winograd_fwd: m = B^T d (per column), then V = m B
      f32x2 m[4][4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        f32x2 d[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) d[r] = *reinterpret_cast<const f32x2*>(&sin_[(r * kWgCols + 2 * n + c) * XS + 2 * q]);
        m[0][c] = d[0] - d[2];
        m[1][c] = d[1] + d[2];
        m[2][c] = d[2] - d[1];
        m[3][c] = d[1] - d[3];
      }
      const int ci0 = 2 * q;
      const int kc = ci0 / 32, k = ci0 % 32;
      const int flane = (k / 8) * 16 + n, j0 = k % 8;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        f32x2 vv[4];
        vv[0] = m[r][0] - m[r][2];
        vv[1] = m[r][1] + m[r][2];
        vv[2] = m[r][2] - m[r][1];
        vv[3] = m[r][1] - m[r][3];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          half2v hv = {half_t(vv[b][0]), half_t(vv[b][1])};
          half_t* dst = reinterpret_cast<half_t*>(&sv[((4 * r + b) * KC + kc) * 64 + flane]) + j0;
          *reinterpret_cast<half2v*>(dst) = hv;
        }
      }
    }
    __syncthreads();  // sv complete; sin_ free

    // next group's input: in flight while this group's GEMMs run
    const bool more = grp + 1 < g_end;
    float vn[kPer];
    load_region(more ? grp + 1 : grp, vn);

    if (active) wg_gemm_store<KC>(u, sv, lane, g, bias, a, img, tr, seg);

    if (more) park_region(vn);
    __syncthreads();  // sin_ holds the next region; every wave is done with sv
  }
}


// ------------------------------------------------------- NCHW fp16 fast path
// For NCHW fp16 input with W % 8 == 0 (the benchmark layout).  Input rows arrive
// in LDS by direct global->LDS DMA (global_load_lds_dwordx4: lane l of an
// instruction writes its 16 bytes at M0 + 16 l) as row pairs (pair k = input
// rows 2k-1 and 2k, fp16, 48 columns [32 s - 8, 32 s + 40) per channel row); tile
// row tr reads pairs tr and tr+1, so every input row of a strip is fetched from
// HBM once.  Chunks outside the image are fetched from a 16-byte zero block.
// The DMA and the output stores are issued from inline assembly, so each wave's
// vector-memory stream is exactly the operations its waits count (loads and
// stores retire in order on gfx9).
constexpr int kRowBytes = 96;                  // 48 fp16 columns per staged channel row


// 16-byte global -> LDS DMA for this lane; lds_wave is the wave's LDS base
// (lane l lands at lds_wave + 16 l).  M0 is saved and restored around it.
__device__ __forceinline__ void wg_dma16(const void* src, uint32_t lds_wave) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds_wave))
      : "memory");
}

__device__ __forceinline__ void wg_st16(void* p, half_t v) {
  asm volatile("global_store_short %0, %1, off nt" ::"v"(p), "v"(__builtin_bit_cast(uint16_t, v)) : "memory");
}
__device__ __forceinline__ void wg_st32(void* p, uint32_t v) {
  asm volatile("global_store_dword %0, %1, off nt" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void wg_st128(void* p, f32x4 v) {
  asm volatile("global_store_dwordx4 %0, %1, off nt\n\ts_nop 0" ::"v"(p), "v"(v) : "memory");
}

// s_waitcnt vmcnt(n) for a run-time n (clamped to 63); expcnt / lgkmcnt untouched.
__device__ __forceinline__ void wg_wait_vmcnt(int n) {
  switch (n < 63 ? (n < 0 ? 0 : n) : 63) {
#define RDV_WG_CASE(k) \
  case k:              \
    asm volatile("s_waitcnt vmcnt(" #k ")" ::: "memory"); \
    break;
    RDV_WG_CASE(0) RDV_WG_CASE(1) RDV_WG_CASE(2) RDV_WG_CASE(3) RDV_WG_CASE(4) RDV_WG_CASE(5) RDV_WG_CASE(6)
    RDV_WG_CASE(7) RDV_WG_CASE(8) RDV_WG_CASE(9) RDV_WG_CASE(10) RDV_WG_CASE(11) RDV_WG_CASE(12) RDV_WG_CASE(13)
    RDV_WG_CASE(14) RDV_WG_CASE(15) RDV_WG_CASE(16) RDV_WG_CASE(17) RDV_WG_CASE(18) RDV_WG_CASE(19)
    RDV_WG_CASE(20) RDV_WG_CASE(21) RDV_WG_CASE(22) RDV_WG_CASE(23) RDV_WG_CASE(24) RDV_WG_CASE(25)
    RDV_WG_CASE(26) RDV_WG_CASE(27) RDV_WG_CASE(28) RDV_WG_CASE(29) RDV_WG_CASE(30) RDV_WG_CASE(31)
    RDV_WG_CASE(32) RDV_WG_CASE(33) RDV_WG_CASE(34) RDV_WG_CASE(35) RDV_WG_CASE(36) RDV_WG_CASE(37)
    RDV_WG_CASE(38) RDV_WG_CASE(39) RDV_WG_CASE(40) RDV_WG_CASE(41) RDV_WG_CASE(42) RDV_WG_CASE(43)
    RDV_WG_CASE(44) RDV_WG_CASE(45) RDV_WG_CASE(46) RDV_WG_CASE(47) RDV_WG_CASE(48) RDV_WG_CASE(49)
    RDV_WG_CASE(50) RDV_WG_CASE(51) RDV_WG_CASE(52) RDV_WG_CASE(53) RDV_WG_CASE(54) RDV_WG_CASE(55)
    RDV_WG_CASE(56) RDV_WG_CASE(57) RDV_WG_CASE(58) RDV_WG_CASE(59) RDV_WG_CASE(60) RDV_WG_CASE(61)
    RDV_WG_CASE(62)
#undef RDV_WG_CASE
    default:
      asm volatile("s_waitcnt vmcnt(63)" ::: "memory");
      break;
  }
}

// f(integral_constant<int, I>) for I = 0 .. N-1, in order, at compile time.
template <class F, int... I>
__device__ __forceinline__ void wg_static_for(std::integer_sequence<int, I...>, F&& f) {
  (f(std::integral_constant<int, I>{}), ...);
}

// LDS reads issued from inline assembly, so the compiler neither sinks them to
// their use nor waits for them itself: the GEMM role, which issues them, waits
// with s_waitcnt lgkmcnt and names the registers it completes (no use of them
// can be scheduled above the wait).  That role issues no other LDS read, and
// keeps at most 15 in flight (the counter's range).
template <int OFF>
__device__ __forceinline__ half8 wg_lds_frag(uint32_t addr) {
  half8 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}
template <int N, int KC>
__device__ __forceinline__ void wg_lds_wait(half8 (&f)[2][KC]) {
  if constexpr (KC == 2)
    asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(f[0][0]), "+v"(f[0][1]), "+v"(f[1][0]), "+v"(f[1][1]) : "i"(N) : "memory");
  else
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(f[0][0]), "+v"(f[1][0]) : "i"(N) : "memory");
}

// wg_gemm for the pipelined kernel: the same products and inverse transform in
// the same order, with the V fragments read two groups ahead of their use (a
// group: column b = G / 2 of the 4 x 4 domain, rows 2 (G % 2) + 0..1, every kc).
// The operands are swapped (A = V, B = U: the two fragment layouts are the
// same), so D is [tile][channel]: lane l holds tiles 4 (l / 16) + 0..3 of
// channel 16 g + l % 16, and a lane's outputs of one row are 8 consecutive
// columns of one channel.
template <int KC>
__device__ __forceinline__ void wg_gemm_pipe(const half8 (&u)[16][KC], const half8* sv, int lane, f32x4 (&yv)[2][2]) {
  const uint32_t addr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sv + lane));
  half8 fr[3][2][KC];
  f32x4 y00, y01, y10, y11, ma[4];
  auto issue = [&](auto gc) {
    constexpr int G = decltype(gc)::value, b = G / 2, ra0 = 2 * (G % 2);
    half8(&f)[2][KC] = fr[G % 3];
    wg_static_for(std::make_integer_sequence<int, 2 * KC>{}, [&](auto ic) {
      constexpr int r = decltype(ic)::value / KC, kc = decltype(ic)::value % KC;
      f[r][kc] = wg_lds_frag<((4 * (ra0 + r) + b) * KC + kc) * 1024>(addr);
    });
  };
  issue(std::integral_constant<int, 0>{});
  issue(std::integral_constant<int, 1>{});
  wg_static_for(std::make_integer_sequence<int, 8>{}, [&](auto gc) {
    constexpr int G = decltype(gc)::value, b = G / 2, ra0 = 2 * (G % 2);
    if constexpr (G + 2 < 8) {
      issue(std::integral_constant<int, G + 2>{});
      wg_lds_wait<4 * KC, KC>(fr[G % 3]);
    } else if constexpr (G + 1 < 8) {
      wg_lds_wait<2 * KC, KC>(fr[G % 3]);
    } else {
      wg_lds_wait<0, KC>(fr[G % 3]);
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      f32x4 acc = {};
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(fr[G % 3][r][kc], u[4 * (ra0 + r) + b][kc], acc, 0, 0, 0);
      ma[ra0 + r] = acc;
    }
    if constexpr (G % 2 == 1) {
      const f32x4 t0 = ma[0] + ma[1] + ma[2];
      const f32x4 t1 = ma[1] - ma[2] - ma[3];
      if constexpr (b == 0) {
        y00 = t0;
        y10 = t1;
      } else if constexpr (b == 1) {
        y00 += t0;
        y01 = t0;
        y10 += t1;
        y11 = t1;
      } else if constexpr (b == 2) {
        y00 += t0;
        y01 -= t0;
        y10 += t1;
        y11 -= t1;
      } else {
        y01 -= t0;
        y11 -= t1;
      }
    }
  });
  yv[0][0] = y00;
  yv[0][1] = y01;
  yv[1][0] = y10;
  yv[1][1] = y11;
}

// ------------------------------------------------------- pipelined kernel
// winograd3x3_pipe_kernel: each 8-wave block (one per CU) walks a vertical strip
// of one image, 32 output columns (16 tiles) by rows_per_item tile rows, top to
// bottom, in two roles of 4 waves, so that a tile row's input transform runs
// while the previous row's GEMMs and stores run:
//   waves 4-7 (input role): row pairs into a 4-slot ring by DMA (3 pairs
//     ahead), then V of tile row s into sv buffer s % 2;
//   waves 0-3 (GEMM role): U in registers (its loads run under the first V
//     transform, and the first tile row's GEMMs start on each group of U as it
//     lands); the GEMMs, inverse transform and stores of tile row s - 1 from sv
//     buffer (s - 1) % 2.
// Step s = 0 .. R ends with one barrier.  Each role's vector-memory stream is
// its own (DMAs only; U's loads then stores only), so the input role's waits
// count its DMA instructions alone.  The V transform runs on the matrix cores:
// one v_mfma_f32_16x16x16_f16 per (channel, 16 tiles) multiplies the patches by
// the 16 x 16 matrix of B^T (x) B^T (entries 0 and +-1, so the products are
// exact), and each lane rounds its 4 positions x 8 channels to fp16 and writes
// 4 B fragments.  Each V value is a sum of four +-d terms.  The reference forms
// it as (d_i +- d_j) +- (d_k +- d_l) in fp32; both give the same fp32 value
// whenever the partial sums are exact, which holds when the four fp16 inputs
// lie within a factor 2^12 of each other (or are zero).  Otherwise the two can
// differ by fp32 rounding before V's fp16 rounding.
constexpr int kPipeSlots = 4;
template <int KC>
struct WgPipeLds {
  static constexpr int kSlotBytes = 2 * 32 * KC * kRowBytes;
  static constexpr int kSvHalf8 = 16 * KC * 64;
  static constexpr int kBytes = kPipeSlots * kSlotBytes + 2 * kSvHalf8 * 16;
  // the ring is the DMA target (M0 addresses): it starts the block and must end below 64 KiB
  static_assert(kPipeSlots * kSlotBytes <= 65536, "DMA ring past 64 KiB");
};

template <int KC>
__global__ __launch_bounds__(512, 1) void winograd3x3_pipe_kernel(WinogradArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  using LD = WgPipeLds<KC>;
  constexpr int CH = 32 * KC;                          // staged channels
  constexpr int kPairChunks = 2 * CH * 6;              // 16-byte chunks per row pair (multiple of 64)
  constexpr int kLoads = (kPairChunks + 255) / 256;    // DMA rounds per pair
  constexpr int kSlotBytes = LD::kSlotBytes;
  uint32_t* const ring = reinterpret_cast<uint32_t*>(smem);
  half8* const svb = reinterpret_cast<half8*>(smem + kPipeSlots * kSlotBytes);
  const int tid = int(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  __builtin_assume(wave >= 0 && wave < 8);
  const int role = wave >> 2, w = wave & 3;
  const int hw = a.H * a.W;
  const half_t* __restrict__ x = static_cast<const half_t*>(a.x);

  auto decode = [&](int64_t item, int& img, int& seg, int& tr0) {
    const int chunk = int(item % a.chunks);
    const int64_t strip = item / a.chunks;
    seg = int(strip % a.seg);
    img = int(strip / a.seg);
    tr0 = chunk * a.rows_per_item;
  };

  if (role == 1) {
    // ================= input role
    const uint32_t ring_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(ring));
    int Ld = 0;  // this wave's DMA instructions per pair
#pragma unroll
    for (int i = 0; i < kLoads; ++i) Ld += (i * 256 + w * 64 < kPairChunks) ? 1 : 0;
    auto dma_pair = [&](int img, int seg, int k, int slot) {
      const half_t* base = x + int64_t(img) * a.cin * hw;
#pragma unroll
      for (int i = 0; i < kLoads; ++i) {
        const int first = i * 256 + w * 64;  // wave-uniform
        if (first < kPairChunks) {
          const int lin = first + lane;
          const int cc = lin % 6;
          const int rest = lin / 6;
          const int ci = rest % CH;
          const int row = 2 * k - 1 + rest / CH;
          const int col = 32 * seg - 8 + 8 * cc;
          const bool ok = (ci < a.cin) & (row >= 0) & (row < a.H) & (col >= 0) & (col < a.W);
          const void* src = ok ? static_cast<const void*>(base + (ci * a.H + row) * a.W + col)
                               : static_cast<const void*>(g_wg_zero16);
          wg_dma16(src, ring_lds + uint32_t(slot * kSlotBytes + first * 16));
        }
      }
    };
    // V = B^T d B as one v_mfma_f32_16x16x16_f16 per channel and 16 tiles:
    // V[p][tile] = sum_k T[p][k] d[k][tile] with p = 4a + b the transform-domain
    // position, k = 4i + j the patch position (row i, column j) and
    // T[p][k] = B^T[a][i] B^T[b][j] in {0, +-1}.  Lane (q, n) holds the A row
    // p = n, columns k = 4q .. 4q + 3 of T; the B column of tile n, patch row q;
    // and D rows p = 4q .. 4q + 3 of tile n.
    const int n = lane & 15, qr = lane >> 4;
    half4 tfrag;
    {
      // B^T = {{1, 0, -1, 0}, {0, 1, 1, 0}, {0, -1, 1, 0}, {0, 1, 0, -1}}, entry
      // (r, c) as a 2-bit two's-complement field at bit 2 (4 r + c)
      auto bt = [](int r, int c) { return int(0xc41c1431u << (30 - 2 * (4 * r + c))) >> 30; };
      const int a0 = n >> 2, b0 = n & 3;
#pragma unroll
      for (int j = 0; j < 4; ++j) tfrag[j] = half_t(float(bt(a0, qr) * bt(b0, j)));
    }
    for (int64_t item = blockIdx.x; item < a.items; item += gridDim.x) {
      int img, seg, tr0;
      decode(item, img, seg, tr0);
      const int R = min(a.rows_per_item, a.th - tr0);  // tile rows (>= 1); pairs 0..R
      for (int q = 0; q < min(3, R + 1); ++q) dma_pair(img, seg, tr0 + q, q);
      wg_wait_vmcnt(2 <= R ? Ld : 0);  // pairs 0 and 1 landed (pair 2 may be in flight)
      __syncthreads();
      for (int s = 0; s <= R; ++s) {
        if (s < R) {
          // ---- V = B^T d B of tile row s (pairs s, s + 1): wave w transforms the
          // 8-channel groups w, w + 4, .. of the 16 tiles.  Columns 2n-1 .. 2n+2 of
          // tile n are halves 2n+7 .. 2n+10 of a staged row = the high half of dword
          // n+3, dword n+4 and the low half of dword n+5; patch rows 0, 1 are rows
          // of pair s (slot sa), rows 2, 3 of pair s + 1 (slot sb).
          {
            const int sa = s % kPipeSlots, sb = (s + 1) % kPipeSlots;
            const uint32_t* rowp = reinterpret_cast<const uint32_t*>(
                                       smem + (qr < 2 ? sa : sb) * kSlotBytes + (qr & 1) * CH * kRowBytes) +
                                   n + 3;
            half8* sv = svb + (s & 1) * LD::kSvHalf8;
            const f32x4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int gi = 0; gi < CH / 32; ++gi) {
              const int c0 = 8 * (w + 4 * gi);  // the group's first channel
              f32x4 vacc[8];
#pragma unroll
              for (int cc = 0; cc < 8; ++cc) {
                const uint32_t* rp = rowp + (c0 + cc) * (kRowBytes / 4);
                const uint32_t d0 = rp[0], d1 = rp[1], d2 = rp[2];
                const uint32_t lo = __builtin_amdgcn_alignbit(d1, d0, 16);  // columns 0, 1
                const uint32_t hi = __builtin_amdgcn_alignbit(d2, d1, 16);  // columns 2, 3
                const half4 bfrag = __builtin_bit_cast(half4, (uint32_t __attribute__((ext_vector_type(2)))){lo, hi});
                vacc[cc] = __builtin_amdgcn_mfma_f32_16x16x16f16(tfrag, bfrag, zero4, 0, 0, 0);
              }
              // lane (qr, n): positions 4 qr + j of tile n for the group's 8 channels,
              // rounded to fp16: one B fragment (8 consecutive channels) per position
              const int kc = c0 / 32, flane = ((c0 % 32) / 8) * 16 + n;
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                half8 h;
#pragma unroll
                for (int cc = 0; cc < 8; ++cc) h[cc] = half_t(vacc[cc][j]);
                sv[((4 * qr + j) * KC + kc) * 64 + flane] = h;
              }
            }
          }
          // pair s + 3 into the slot pair s - 1 used (read by step s - 1, before its barrier)
          if (s + 3 <= R) dma_pair(img, seg, tr0 + s + 3, (s + 3) % kPipeSlots);
          // pair s + 2 landed for the next step (only pair s + 3 may still be in flight)
          if (s + 2 <= R) wg_wait_vmcnt(s + 3 <= R ? Ld : 0);
        }
        __syncthreads();
      }
    }
    return;
  }

  // ================= GEMM role: wave w owns output channels 16 (4 blockIdx.y + w) + 0..15
  const int g = blockIdx.y * 4 + w;
  const bool active = 16 * g < a.cout;
  // Bias, ReLU and the stores of tile row tr's outputs yv (after wg_gemm_pipe):
  // lane (q, c) holds channel co = 16 g + c of tiles 4 q + 0..3 of the strip.
  // W % 8 == 0, so those four tiles are all inside the image or all outside.
  const int co = 16 * g + (lane & 15);
  auto finish_row = [&](f32x4 (&yv)[2][2], float bias, int img, int seg, int tr) {
    const int tq = seg * kWgTiles + 4 * (lane >> 4);  // the lane's first tile
    if (tq >= a.W / 2) return;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int jx = 0; jx < 2; ++jx) yv[i][jx] += bias;
    const int hw = a.H * a.W;
    if (a.out_layout == RDV_LAYOUT_CHW) {
      const int64_t o = (int64_t(img) * a.cout + co) * hw + int64_t(2 * tr) * a.W + 2 * tq;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        if (a.out_dtype == RDV_DTYPE_F16) {
          // ReLU after the fp16 rounding, two values per instruction (max(x, 0)
          // commutes with a monotonic rounding that maps 0 to 0)
          uint32_t hv[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) hv[j] = __builtin_bit_cast(uint32_t, half2v{half_t(yv[i][0][j]), half_t(yv[i][1][j])});
          if (a.relu) {
            // volatile: a branch on the uniform flag, not a per-lane select of both results
#pragma unroll
            for (int j = 0; j < 4; ++j) asm volatile("v_pk_max_f16 %0, %1, 0" : "=v"(hv[j]) : "v"(hv[j]));
          }
          wg_st128(static_cast<half_t*>(a.y) + o + int64_t(i) * a.W, __builtin_bit_cast(f32x4, hv));
        } else {
          f32x4 v0, v1;
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            v0[2 * j] = yv[i][0][j];
            v0[2 * j + 1] = yv[i][1][j];
            v1[2 * j] = yv[i][0][j + 2];
            v1[2 * j + 1] = yv[i][1][j + 2];
          }
          if (a.relu) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              v0[e] = fmaxf(v0[e], 0.0f);
              v1[e] = fmaxf(v1[e], 0.0f);
            }
          }
          float* dst = static_cast<float*>(a.y) + o + int64_t(i) * a.W;
          wg_st128(dst, v0);
          wg_st128(dst + 4, v1);
        }
      }
    } else {
      // channels-last: one element per (pixel, channel); the 16 lanes of a tile
      // quad write 16 consecutive channels of each pixel
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int jx = 0; jx < 2; ++jx) {
            float v = yv[i][jx][j];
            if (a.relu) v = fmaxf(v, 0.0f);
            const int64_t o = (int64_t(img) * hw + int64_t(2 * tr + i) * a.W + 2 * (tq + j) + jx) * a.cout + co;
            if (a.out_dtype == RDV_DTYPE_F16) wg_st16(static_cast<half_t*>(a.y) + o, half_t(v));
            else wg_st32(static_cast<float*>(a.y) + o, __builtin_bit_cast(uint32_t, v));
          }
    }
  };
  // The GEMMs, inverse transform, bias, ReLU and stores of tile row tr from sv buffer `buf`.
  auto gemm_row = [&](const half8 (&uu)[16][KC], float bias, int img, int seg, int tr, int buf) {
    f32x4 yv[2][2];
    wg_gemm_pipe(uu, svb + buf * LD::kSvHalf8, lane, yv);
    finish_row(yv, bias, img, seg, tr);
  };
  // U's loads are issued after the first item's first barrier (its first pairs
  // landed), so the input role's DMAs go first, and they run under the input
  // role's V of tile row 0, which needs no U.  The bias comes first and U in the
  // order of wg_gemm_pipe's fragment groups (column b = G / 2, rows 2 (G % 2) +
  // 0..1), and the first tile row is peeled out of the loop below: the
  // compiler's per-register waits then let each group's MFMAs start as soon as
  // that group's U has landed, instead of after all 128 KiB of it.  Those waits
  // count only these loads (no store is issued before that row's GEMMs), and the
  // peeled row uses every U register and the bias, so nothing is pending for the
  // compiler inside the loop.
  const bool any = int64_t(blockIdx.x) < a.items;
  if (any) __syncthreads();
  const int g_n = (a.cout + 15) / 16;
  const int gu = active ? g : 0;
  // this lane's channel bias (unconditional load: a zero block for a null bias, or a clamped index)
  const float* bsrc = a.bias ? a.bias : reinterpret_cast<const float*>(g_wg_zero16);
  const float bias = bsrc[a.bias && co < a.cout ? co : 0];
  half8 u[16][KC];
  wg_static_for(std::make_integer_sequence<int, 8>{}, [&](auto gc) {
    constexpr int G = decltype(gc)::value, b = G / 2, ra0 = 2 * (G % 2);
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        const int p = 4 * (ra0 + r) + b;
        u[p][kc] = reinterpret_cast<const half8*>(a.U)[((int64_t(p) * KC + kc) * g_n + gu) * 64 + lane];
      }
  });
  if (!any) return;
  __syncthreads();  // end of the first item's step 0 (V of its first tile row in sv buffer 0)
  {
    int img, seg, tr0;
    decode(blockIdx.x, img, seg, tr0);
    // step 1 of the first item
    f32x4 yv[2][2] = {};
    if (active) wg_gemm_pipe(u, svb, lane, yv);
    // every path uses U and the bias here, before any store, so none enters the
    // loop with a load pending for the compiler (it would wait there, on the
    // stores); on the active path every load has already been waited for
#pragma unroll
    for (int p = 0; p < 16; ++p)
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) asm volatile("" ::"v"(u[p][kc]));
    asm volatile("" ::"v"(bias));
    if (active) finish_row(yv, bias, img, seg, tr0);
    __syncthreads();
  }
  for (int64_t item = blockIdx.x; item < a.items; item += gridDim.x) {
    int img, seg, tr0;
    decode(item, img, seg, tr0);
    const int R = min(a.rows_per_item, a.th - tr0);
    const int s0 = item == blockIdx.x ? 2 : 0;  // the first item's steps 0 and 1 are above
    if (s0 == 0) __syncthreads();               // the input role's first two pairs
    for (int s = s0; s <= R; ++s) {
      if (s >= 1 && active) gemm_row(u, bias, img, seg, tr0 + s - 1, (s - 1) & 1);
      __syncthreads();
    }
  }
}

int64_t winograd_weight_bytes(int cin, int cout) {
  const int kc_n = (cin + 31) / 32, g_n = (cout + 15) / 16;
  return int64_t(16) * kc_n * g_n * 64 * 8 * 2;
}

int launch_winograd_transform_weight(const void* w, int w_layout, int w_dtype, int cin, int cout, void* U,
                                     hipStream_t stream) {
  const int kc_n = (cin + 31) / 32, g_n = (cout + 15) / 16;
  const int64_t total = int64_t(16) * kc_n * g_n * 64 * 8;
  winograd_transform_weight_kernel<<<dim3(unsigned((total + 255) / 256)), dim3(256), 0, stream>>>(
      w, w_layout, w_dtype, cin, cout, kc_n, g_n, static_cast<half_t*>(U));
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

int launch_winograd3x3(const rdv_conv_desc& d, const void* x, const void* U, const float* bias, void* y,
                       hipStream_t stream) {
  DeviceInfo di;
  int rc = device_info(&di);
  if (rc != RDV_OK) return rc;
  WinogradArgs a;
  a.x = x;
  a.U = static_cast<const half_t*>(U);
  a.bias = bias;
  a.y = y;
  a.batch = d.batch;
  a.H = d.H;
  a.W = d.W;
  a.cin = d.cin;
  a.cout = d.cout;
  a.in_layout = d.in_layout;
  a.in_dtype = d.in_dtype;
  a.out_layout = d.out_layout;
  a.out_dtype = d.out_dtype;
  a.relu = d.relu;
  a.th = d.H / 2;
  a.seg = (d.W / 2 + kWgTiles - 1) / kWgTiles;
  a.ngroups = int64_t(d.batch) * a.th * a.seg;
  if (a.ngroups == 0) return RDV_OK;
  const int groups16 = (d.cout + 15) / 16;
  const int slices = (groups16 + 3) / 4;  // 64-channel slices (grid y)
  const bool f16 = d.in_dtype == RDV_DTYPE_F16, chw = d.in_layout == RDV_LAYOUT_CHW;
  // the pipelined kernel reads x and writes y with 16-byte vector accesses; other buffers take the strip kernel
  if (f16 && chw && d.W % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
      reinterpret_cast<uintptr_t>(y) % 16 == 0) {
    // pipelined kernel: one 8-wave block per CU, each walking rows_per_item tile rows of a strip
    static bool attr = false;
    if (!attr) {
      RDV_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&winograd3x3_pipe_kernel<1>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, WgPipeLds<1>::kBytes));
      RDV_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&winograd3x3_pipe_kernel<2>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, WgPipeLds<2>::kBytes));
      attr = true;
    }
    const int64_t strips = int64_t(d.batch) * a.seg;
    const int64_t target = std::max<int64_t>(1, di.cu_count / slices);
    const int64_t per_strip = std::max<int64_t>(1, target / strips);
    a.rows_per_item = int((a.th + per_strip - 1) / per_strip);
    a.chunks = (a.th + a.rows_per_item - 1) / a.rows_per_item;
    a.items = strips * a.chunks;
    const int64_t blocks = std::min<int64_t>(a.items, target);
    const dim3 grid(static_cast<unsigned>(blocks), static_cast<unsigned>(slices)), block(512);
    if (d.cin <= 32) winograd3x3_pipe_kernel<1><<<grid, block, WgPipeLds<1>::kBytes, stream>>>(a);
    else winograd3x3_pipe_kernel<2><<<grid, block, WgPipeLds<2>::kBytes, stream>>>(a);
    RDV_HIP_TRY(hipGetLastError());
    return RDV_OK;
  }
  int64_t blocks = (2 * int64_t(di.cu_count) + slices - 1) / slices;  // ~2 resident blocks per CU
  if (a.ngroups < blocks) blocks = a.ngroups;
  const dim3 grid(static_cast<unsigned>(blocks), static_cast<unsigned>(slices)), block(256);
  if (d.cin <= 32) {
    if (f16) {
      if (chw) winograd3x3_kernel<1, true, true><<<grid, block, 0, stream>>>(a);
      else winograd3x3_kernel<1, true, false><<<grid, block, 0, stream>>>(a);
    } else {
      if (chw) winograd3x3_kernel<1, false, true><<<grid, block, 0, stream>>>(a);
      else winograd3x3_kernel<1, false, false><<<grid, block, 0, stream>>>(a);
    }
  } else {
    if (f16) {
      if (chw) winograd3x3_kernel<2, true, true><<<grid, block, 0, stream>>>(a);
      else winograd3x3_kernel<2, true, false><<<grid, block, 0, stream>>>(a);
    } else {
      if (chw) winograd3x3_kernel<2, false, true><<<grid, block, 0, stream>>>(a);
      else winograd3x3_kernel<2, false, false><<<grid, block, 0, stream>>>(a);
    }
  }
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

}  // namespace rdv
