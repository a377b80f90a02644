// Direct 2-D convolution of any KH x KW kernel, stride 1, 'same' zero padding
// (pad = K / 2 on the top and left, as the reference's kernels index it), over
// channels-last fp32 images: y[H*W, COUT] = conv(x[H*W, CIN], w) + bias.
//
// Replaces the dispatches of Conv2DTensorOp (fp32, src/rdv/domain/nn.py:414-470,
// src/rdv/shaders/tensors/conv2d_tensor_op.h:20-80), and of the fp16-operand
// variants Conv2DTensorOpFast (nn.py:608-668, conv2d_tensor_op_fast.h),
// Conv2DTensorOpSimple (nn.py:669-756, conv2d_tensor_op_simple.h),
// Conv2DTensorOpSimple3x3 (nn.py:757-850, conv2d_tensor_op_simple3x3.h) and
// Conv2DTensorOpWindow3x3 (nn.py:851-1000, conv2d_tensor_op_window3x3.h).  The
// four fp16 variants compute one function -- x and w rounded to fp16, products
// summed in fp32 over K = KH KW CIN, fp32 bias -- and differ only in tiling,
// so one kernel serves them; the fp32 op is the same kernel on fp32 matrix
// cores.  The reference's sum order (taps in (kh, kw) order, channels
// ascending) is the order of the K index here; only the fp32 association
// inside the matrix cores differs.
//
// MI355X mapping: implicit GEMM.  M = the H W output pixels, N = COUT, K = the
// KH KW CIN taps-and-channels.  A block of 4 waves owns one block of <= 128
// output channels for the whole launch and stages that block of w into LDS
// once, converted to fp16 (or kept fp32) in MFMA-fragment order; its waves
// then walk 32-pixel tiles with a grid stride.  Per K chunk a lane gathers 8
// (fp16) or 4 (fp32) consecutive channels of one tap of one pixel straight
// from x -- the im2col matrix is never formed -- and the next chunk's loads are
// issued before the current chunk's MFMAs.  Taps outside the image and K past
// KH KW CIN read a clamped address and are zeroed on conversion, so every load
// is in bounds and unconditional (channel counts that are not a multiple of
// the lane's group take a per-element gather and scalar stores instead).
// Neighbouring taps re-read neighbouring pixels, which the L2 serves (a tile's
// receptive field is a few image rows).
//   fp16: v_mfma_f32_16x16x32_f16, A = w[16 out][32 k], B = x^T[32 k][16 px]
//   fp32: v_mfma_f32_16x16x4f32 over 16-k chunks (a lane's float4 feeds 4 MFMAs)
// When a block of w exceeds the LDS budget it is restaged per K pass per tile.
#include <algorithm>

#include "rdv_common.h"

namespace rdv {

namespace {

constexpr int kCvThreads = 256;
constexpr int kCvWaves = kCvThreads / 64;
constexpr int kCvRT = 2;            // 16-pixel subtiles per wave
constexpr int kCvMaxOb = 128;       // output channels per block
constexpr int64_t kCvLdsCap = 144 * 1024;

struct ConvArgs {
  const float* x;     // [H W, cin]
  const float* w;     // RSCK [kh][kw][cin][cout] or KCRS [cout][cin][kh][kw], fp32
  const float* bias;  // [cout] or null
  float* y;           // [H W, cout]
  int64_t rows;       // H W
  int64_t tasks;      // pixel tiles of kCvWaves * 16 * kCvRT
  int H, W, cin, cout, kh, kw, ph, pw;
  int K;              // kh kw cin
  int wlayout, relu;
  int kp;             // K per LDS pass (multiple of the chunk width)
  int passes;
  int ob, n_ob;
  int w_rows;         // RSCK with 16-byte rows: cv_stage_rows
};

template <bool F16>
struct CvStep;
template <>
struct CvStep<true> {
  static constexpr int kK = 32;   // K per chunk
  static constexpr int kLane = 8; // consecutive channels per lane
};
template <>
struct CvStep<false> {
  static constexpr int kK = 16;
  static constexpr int kLane = 4;
};

__device__ __forceinline__ float w_at(const ConvArgs& a, int o, int k) {
  // k = tap * cin + ci, tap = kh * KW + kw
  if (a.wlayout == RDV_WLAYOUT_RSCK) return a.w[int64_t(k) * a.cout + o];
  const int tap = k / a.cin, ci = k - tap * a.cin;
  return a.w[(int64_t(o) * a.cin + ci) * (a.kh * a.kw) + tap];
}

// Physical position of slot ln (0..63) of output tile t's filter fragment in
// LDS: the two low bits XOR (ln / 16 + t) % 4.  The staging writes of a wave
// (slots 16 kq + 4 j + e of every t and kq for one e) then spread over every
// bank instead of four (a 16-way conflict), and a fragment's 64 slots stay a
// permutation of themselves, so its reads (lane l reads slot l) remain
// conflict-free.
__device__ __forceinline__ int cv_swz(int t, int ln) { return ln ^ (((ln >> 4) + t) & 3); }

// w block [o0, o0 + ob) x K [k0, k0 + kp) into LDS, fragment order: slot
// ((t * nkc + c) * 64 + lane) = 16 bytes, out o0 + 16 t + lane % 16, K
// k0 + c kK + (lane / 16) kLane + 0 .. kLane-1 (fp16 halves or fp32 floats);
// outputs past cout and K past KH KW CIN are zero.  Also the bias block.
template <bool F16>
__device__ void cv_stage(const ConvArgs& a, int o0, int k0, int nkc, f32x4* sw, float* sb, int tid = -1,
                         int nthr = kCvThreads) {
  using S = CvStep<F16>;
  if (tid < 0) tid = int(threadIdx.x);
  const int nt = a.ob / 16;
  const int slots = nt * nkc * 64;
  for (int s = tid; s < slots; s += nthr) {
    const int t = s / (nkc * 64);
    const int rem = s - t * (nkc * 64);
    const int c = rem >> 6, ln = rem & 63;
    const int o = o0 + 16 * t + (ln & 15);
    const int k = k0 + c * S::kK + (ln >> 4) * S::kLane;
    f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
    if (o < a.cout && k < a.K) {
      // K is a multiple of kLane only when cin is; past K the slots are zero
      if constexpr (F16) {
        half8 h;
#pragma unroll
        for (int i = 0; i < 8; ++i) h[i] = half_t(k + i < a.K ? w_at(a, o, k + i) : 0.0f);
        v = __builtin_bit_cast(f32x4, h);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = k + i < a.K ? w_at(a, o, k + i) : 0.0f;
      }
    }
    sw[(t * nkc + c) * 64 + cv_swz(t, ln)] = v;
  }
  for (int i = tid; i < a.ob; i += nthr) sb[i] = (a.bias != nullptr && o0 + i < a.cout) ? a.bias[o0 + i] : 0.0f;
}

// cv_stage for an RSCK filter whose rows are 16-byte vectors (cout % 4 == 0,
// w 16-byte aligned): w[k][o] is contiguous in o, so a thread reads kLane rows
// k .. k + kLane - 1 of four consecutive outputs (one 16-byte load per row,
// coalesced across threads) and writes the four slots of those outputs.  Same
// slot contents as cv_stage.
template <bool F16>
__device__ void cv_stage_rows(const ConvArgs& a, int o0, int k0, int nkc, f32x4* sw, float* sb) {
  using S = CvStep<F16>;
  const int nt = a.ob / 16;
  const int groups = nt * nkc * 16;  // (t, c, lane / 16, four outputs)
  for (int gi = threadIdx.x; gi < groups; gi += kCvThreads) {
    const int j = gi & 3, kq = (gi >> 2) & 3;
    const int tc = gi >> 4;
    const int t = tc / nkc, c = tc - t * nkc;
    const int o = o0 + 16 * t + 4 * j;
    const int k = k0 + c * S::kK + kq * S::kLane;
    f32x4 r[S::kLane];
#pragma unroll
    for (int i = 0; i < S::kLane; ++i) {
      const bool ok = o < a.cout && k + i < a.K;
      r[i] = ok ? *reinterpret_cast<const f32x4*>(a.w + int64_t(k + i) * a.cout + o) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f32x4 v;
      if constexpr (F16) {
        half8 h;
#pragma unroll
        for (int i = 0; i < 8; ++i) h[i] = half_t(r[i][e]);
        v = __builtin_bit_cast(f32x4, h);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = r[i][e];
      }
      sw[(t * nkc + c) * 64 + cv_swz(t, kq * 16 + 4 * j + e)] = v;
    }
  }
  for (int i = threadIdx.x; i < a.ob; i += kCvThreads)
    sb[i] = (a.bias != nullptr && o0 + i < a.cout) ? a.bias[o0 + i] : 0.0f;
}

template <bool F16>
__device__ __forceinline__ void cv_stage_any(const ConvArgs& a, int o0, int k0, int nkc, f32x4* sw, float* sb) {
  if (a.w_rows) cv_stage_rows<F16>(a, o0, k0, nkc, sw, sb);
  else cv_stage<F16>(a, o0, k0, nkc, sw, sb);
}

// One lane's view of its kCvRT pixels: image coordinates and validity.
struct CvPix {
  int h[kCvRT], w[kCvRT];
  bool live[kCvRT];
};

// Gathers K chunk kk0 (this lane's kLane channels of one tap) for each pixel.
// VEC: cin is a multiple of kLane and x 16-byte aligned, so a lane's kLane
// elements are consecutive channels of one tap (16-byte loads); otherwise
// each element finds its own tap and channel (scalar loads, zero past K).
template <bool F16, bool VEC>
__device__ __forceinline__ void cv_load(const ConvArgs& a, const CvPix& px, int kk0, int q,
                                        f32x4 (&raw)[kCvRT][CvStep<F16>::kLane / 4], bool (&ok)[kCvRT]) {
  using S = CvStep<F16>;
  const int kk = kk0 + q * S::kLane;
  if constexpr (!VEC) {
#pragma unroll
    for (int rr = 0; rr < kCvRT; ++rr) ok[rr] = px.live[rr];
#pragma unroll
    for (int i = 0; i < S::kLane; ++i) {
      const int k = kk + i;
      const int tap = k / a.cin;
      const int ci = k - tap * a.cin;
      const int th = tap / a.kw;
      const int tw = tap - th * a.kw;
#pragma unroll
      for (int rr = 0; rr < kCvRT; ++rr) {
        const int ih = px.h[rr] + th - a.ph, iw = px.w[rr] + tw - a.pw;
        const bool v = k < a.K && ih >= 0 && ih < a.H && iw >= 0 && iw < a.W;
        const float e = a.x[v ? (int64_t(ih) * a.W + iw) * a.cin + ci : 0];
        raw[rr][i >> 2][i & 3] = v ? e : 0.0f;
      }
    }
    return;
  }
  const int tap = kk / a.cin;
  const int ci = kk - tap * a.cin;
  const int th = tap / a.kw;
  const int tw = tap - th * a.kw;
  const bool kin = kk < a.K;
#pragma unroll
  for (int rr = 0; rr < kCvRT; ++rr) {
    const int ih = px.h[rr] + th - a.ph, iw = px.w[rr] + tw - a.pw;
    const bool v = kin && px.live[rr] && ih >= 0 && ih < a.H && iw >= 0 && iw < a.W;
    const int64_t off = v ? (int64_t(ih) * a.W + iw) * a.cin + ci : 0;
    const f32x4* src = reinterpret_cast<const f32x4*>(a.x + off);
#pragma unroll
    for (int j = 0; j < S::kLane / 4; ++j) raw[rr][j] = src[j];
    ok[rr] = v;
  }
}

template <bool F16, int NT>
__device__ __forceinline__ void cv_mma(const f32x4* sw, int nt, int nkc, int c, int lane,
                                       const f32x4 (&raw)[kCvRT][CvStep<F16>::kLane / 4], const bool (&ok)[kCvRT],
                                       f32x4 (&acc)[kCvRT][NT]) {
  if constexpr (F16) {
    half8 xb[kCvRT];
#pragma unroll
    for (int rr = 0; rr < kCvRT; ++rr) {
      half8 hv;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        hv[j] = half_t(raw[rr][0][j]);
        hv[4 + j] = half_t(raw[rr][1][j]);
      }
      xb[rr] = ok[rr] ? hv : half8{};
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t < nt) {
        const half8 wh = __builtin_bit_cast(half8, sw[(t * nkc + c) * 64 + cv_swz(t, lane)]);
#pragma unroll
        for (int rr = 0; rr < kCvRT; ++rr)
          acc[rr][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wh, xb[rr], acc[rr][t], 0, 0, 0);
      }
    }
  } else {
    f32x4 xv[kCvRT];
#pragma unroll
    for (int rr = 0; rr < kCvRT; ++rr) xv[rr] = ok[rr] ? raw[rr][0] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t < nt) {
        const f32x4 wv = sw[(t * nkc + c) * 64 + cv_swz(t, lane)];
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int rr = 0; rr < kCvRT; ++rr)
            acc[rr][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[s], xv[rr][s], acc[rr][t], 0, 0, 0);
      }
    }
  }
}

template <bool F16, int NT, bool VEC>
__global__ __launch_bounds__(kCvThreads) void conv_op_kernel(ConvArgs a) {
  using S = CvStep<F16>;
  extern __shared__ f32x4 cv_smem[];
  const int nt = a.ob / 16;
  const int nkc = a.kp / S::kK;
  f32x4* sw = cv_smem;
  float* sb = reinterpret_cast<float*>(cv_smem + nt * nkc * 64);
  const int lane = threadIdx.x & 63;
  const int q = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // blockIdx.x = pixel workgroup * n_ob + output block: the blocks sharing
  // pixels are dispatched back to back, so their x re-reads hit the cache.
  const int ob_idx = blockIdx.x % a.n_ob;
  const int64_t rwg = blockIdx.x / a.n_ob;
  const int64_t rstride = gridDim.x / a.n_ob;
  const int o0 = ob_idx * a.ob;

  if (a.passes == 1) {
    cv_stage_any<F16>(a, o0, 0, nkc, sw, sb);
    __syncthreads();
  }
  for (int64_t task = rwg; task < a.tasks; task += rstride) {
    CvPix px;
#pragma unroll
    for (int rr = 0; rr < kCvRT; ++rr) {
      const int64_t p = (task * kCvWaves + wave) * (16 * kCvRT) + rr * 16 + (lane & 15);
      px.live[rr] = p < a.rows;
      const int64_t pc = px.live[rr] ? p : 0;
      px.h[rr] = int(pc / a.W);
      px.w[rr] = int(pc - int64_t(px.h[rr]) * a.W);
    }
    f32x4 acc[kCvRT][NT];
    for (int pass = 0; pass < a.passes; ++pass) {
      const int k0 = pass * a.kp;
      if (a.passes > 1) {
        __syncthreads();
        cv_stage_any<F16>(a, o0, k0, nkc, sw, sb);
        __syncthreads();
      }
      if (pass == 0) {
        const f32x4* sb4 = reinterpret_cast<const f32x4*>(sb);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const f32x4 b = t < nt ? sb4[t * 4 + q] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int rr = 0; rr < kCvRT; ++rr) acc[rr][t] = b;
        }
      }
      // chunks in pairs on two register sets: chunk c + 1's gathers are in
      // flight while chunk c is converted and multiplied
      f32x4 ra[kCvRT][S::kLane / 4], rb[kCvRT][S::kLane / 4];
      bool oka[kCvRT], okb[kCvRT];
      cv_load<F16, VEC>(a, px, k0, q, ra, oka);
      for (int c = 0; c < nkc; c += 2) {
        const bool more = c + 1 < nkc;
        if (more) cv_load<F16, VEC>(a, px, k0 + (c + 1) * S::kK, q, rb, okb);
        cv_mma<F16, NT>(sw, nt, nkc, c, lane, ra, oka, acc);
        if (c + 2 < nkc) cv_load<F16, VEC>(a, px, k0 + (c + 2) * S::kK, q, ra, oka);
        if (more) cv_mma<F16, NT>(sw, nt, nkc, c + 1, lane, rb, okb, acc);
      }
    }
#pragma unroll
    for (int rr = 0; rr < kCvRT; ++rr) {
      if (px.live[rr]) {
        const int64_t p = (task * kCvWaves + wave) * (16 * kCvRT) + rr * 16 + (lane & 15);
        float* yr = a.y + p * a.cout;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const int col = o0 + 16 * t + 4 * q;
          if (t < nt && col < a.cout) {
            f32x4 v = acc[rr][t];
            if (a.relu) {
#pragma unroll
              for (int j = 0; j < 4; ++j) v[j] = fmaxf(v[j], 0.0f);
            }
            if constexpr (VEC) {
              *reinterpret_cast<f32x4*>(yr + col) = v;
            } else {
#pragma unroll
              for (int j = 0; j < 4; ++j)
                if (col + j < a.cout) yr[col + j] = v[j];
            }
          }
        }
      }
    }
  }
}

// ------------------------------------------------------------ spatial tiles
// The fp16 path for a filter block that fits LDS next to a haloed input tile
// (cin % 32 == 0, cout = 16 NT <= 128): a block owns TH x TW tiles of output
// pixels in turn.  Each tile's (TH + KH - 1) x (TW + KW - 1) x cin input window
// is converted to fp16 into LDS once (zero outside the image) and every tap
// reads its B fragments from there, so x crosses the load path about
// (TH + KH - 1)(TW + KW - 1) / (TH TW) times instead of KH KW times.  The
// filter is staged once per launch, its loads issued in one round next to the
// first window's, and the next tile's window loads are in flight (in
// registers) while the current tile's MFMAs run.  MFMA wave w (of four)
// computes output rows 2w and 2w + 1 of the tile, 32 columns each (N blocks
// j = 0..3: row 2w + j / 2, columns 16 (j % 2) ..: four blocks share every filter
// fragment read) against every 16-channel output tile; eight MFMA waves of one
// row each measured no faster (their LDS reads per MFMA grow by half).  K runs over taps in (kh, kw) order and 32-channel
// chunks within a tap: the filter staging's K order.
//
// Both stagings are written for few instructions per load, because at one wave
// per SIMD their instruction count, not the memory system, sets the prologue's
// length: filter loads take immediate offsets from one address per 8-row group,
// and window loads are buffer loads whose descriptor covers one image row, so a
// column or row outside the image reads zero with no per-lane test.
constexpr int kTileH = 8;      // output rows per tile
constexpr int kTileW = 32;     // output columns per tile
// Threads per block: 8 waves, two per SIMD, so that the staging's instruction
// latencies overlap -- up to 5 output tiles, where the MFMA waves' registers
// fit in half a SIMD's file; 4 waves above.
template <int NT>
constexpr int ct_threads() { return NT <= 5 ? 512 : 256; }
// waves that run the MFMAs, each on kTileH / ct_math() output rows
template <int NT>
constexpr int ct_math() { return 4; }
// window units per wave held across a tile (a 3x3, 64-channel window has 90)
template <int NT>
constexpr int ct_win_slots() { return (92 + ct_threads<NT>() / 64 - 1) / (ct_threads<NT>() / 64); }
constexpr int kFiltA = 3;        // filter groups per thread in the first round (64 -> 64 3x3: 2.25 in all)
constexpr int kFiltB = 2;        // filter groups per thread in each later round

struct TileArgs {
  ConvArgs c;
  int tiles_w, tiles;  // column tiles per row band, tiles in all
  int win_w, win_h;    // input window: kTileW + kw - 1, kTileH + kh - 1
  int ps;              // LDS bytes per window pixel: 2 cin + 16 (spreads a wave's reads over every bank)
  int win_bytes;       // window bytes, rounded up to 16, plus 16 spare bytes at the end
  int rp;              // 16-byte fp32 pieces per window row: win_w cin / 4
  int upr;             // 64-piece units per window row: ceil(rp / 64), >= 4
  int units;           // units per window: win_h upr
  int row_bytes;       // bytes per image row: W cin 4 (< 2^31)
  unsigned cq_magic;   // ceil(2^32 / (cin / 4)): p / (cin / 4) == umulhi(p, cq_magic) for every p < rp
  unsigned upr_magic;  // ceil(2^32 / upr): u / upr == umulhi(u, upr_magic) for every unit index u used
  int stage_out;       // output rows staged through the window's LDS (2 NT KiB per wave fit in it)
};

// The RSCK filter (16 NT outputs, every K row) into LDS in fragment order
// (slot (t nkc + c) 64 + lane as cv_stage_rows writes it) plus the bias.
// Group gi: outputs 4 cg .. 4 cg + 3 (cg = gi % 4 NT: tile t = cg / 4, j = cg % 4)
// of K rows 8 rb .. 8 rb + 7 (rb = gi / 4 NT: chunk c = rb / 4, kq = rb % 4) --
// eight 16-byte loads at a fixed stride from one address, transposed in
// registers into four lanes' 8-row fragments.  A round gives each thread NB
// groups: group g0 + u THREADS + tid of round g0.  Every block reads the same
// filter at the same time: each starts at its own row block (a rotation `rot`
// of the group index), so that the blocks of an XCD spread their requests over
// the L2 channels instead of queueing on the same lines.  Past the last group a
// thread takes the last one again: it loads and writes the same bytes as that
// group's owner, so no test guards the conversion (one that the compiler sinks
// the loads below, behind a full wait).
template <int THREADS>
struct CtFilter {
  int groups, rot, nkc;
  __device__ int group(int g0, int u) const {
    const int gi = min(g0 + u * THREADS + int(threadIdx.x), groups - 1) + rot;
    return gi < groups ? gi : gi - groups;
  }
};

template <int NT, int NB, class F>
__device__ __forceinline__ void ct_filter_issue(const F& f, const float* __restrict__ w, int g0,
                                                f32x4 (&r)[NB][8]) {
  constexpr int kG = 4 * NT, kRow = 16 * NT;
#pragma unroll
  for (int u = 0; u < NB; ++u) {
    const int gi = f.group(g0, u);
    const float* src = w + ((gi / kG) * 8 * kRow + 4 * (gi % kG));
#pragma unroll
    for (int i = 0; i < 8; ++i) r[u][i] = *reinterpret_cast<const f32x4*>(src + i * kRow);
  }
}

template <int NT, int NB, class F>
__device__ __forceinline__ void ct_filter_convert(const F& f, int g0, const f32x4 (&r)[NB][8], f32x4* sw) {
  constexpr int kG = 4 * NT;
#pragma unroll
  for (int u = 0; u < NB; ++u) {
    const int gi = f.group(g0, u);
    const int cg = gi % kG, rb = gi / kG;
    const int t = cg >> 2, j = cg & 3, kq = rb & 3, c = rb >> 2;
    const int s = (kq + t) & 3;  // cv_swz's XOR of the slot's two low bits
    f32x4* dst = sw + (t * f.nkc + c) * 64 + kq * 16 + 4 * j;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      half8 h;
#pragma unroll
      for (int i = 0; i < 8; ++i) h[i] = half_t(r[u][i][e]);
      dst[e ^ s] = __builtin_bit_cast(f32x4, h);
    }
  }
}

// The filter's first round (kFiltA groups per thread), then `mid` (the first
// window's loads), then that round's conversion, then rounds of kFiltB groups:
// the first round and the window together fill the registers, and the later
// rounds' loads run while the window's are still in flight.
template <int NT, class Mid>
__device__ void ct_stage_filter(const float* __restrict__ w, const float* __restrict__ bias, int nkc, f32x4* sw,
                                float* sb, Mid&& mid) {
  constexpr int kRow = 16 * NT;  // floats per K row
  constexpr int kThreads = ct_threads<NT>();
  static_assert(kRow <= kThreads, "one bias per thread");
  const int tid = int(threadIdx.x);
  // the bias first: the oldest load, so that waiting for it waits for nothing else
  const float bv = (tid < kRow && bias != nullptr) ? bias[tid] : 0.0f;
  CtFilter<kThreads> f;
  f.groups = nkc * 16 * NT;
  f.rot = int(blockIdx.x * 7u % unsigned(4 * nkc)) * (4 * NT);
  f.nkc = nkc;
  {
    f32x4 r[kFiltA][8];
    ct_filter_issue<NT>(f, w, 0, r);
    __builtin_amdgcn_sched_barrier(0);
    mid();
    ct_filter_convert<NT>(f, 0, r, sw);
  }
  for (int g0 = kFiltA * kThreads; g0 < f.groups; g0 += kFiltB * kThreads) {
    f32x4 r[kFiltB][8];
    ct_filter_issue<NT>(f, w, g0, r);
    ct_filter_convert<NT>(f, g0, r, sw);
  }
  if (tid < kRow) sb[tid] = bv;
}

template <int NT>
__global__ __launch_bounds__(ct_threads<NT>(), 1) void conv_tile_kernel(TileArgs ta) {
  constexpr int kCtWaves = ct_threads<NT>() / 64, kWinSlots = ct_win_slots<NT>();
  constexpr int kMath = ct_math<NT>(), kRows = kTileH / kMath, kNB = 2 * kRows;  // MFMA waves, their rows, N blocks
  const ConvArgs& a = ta.c;
  extern __shared__ f32x4 cv_smem[];
  const int nkc = a.K / 32;
  uint8_t* win = reinterpret_cast<uint8_t*>(cv_smem);
  f32x4* sw = reinterpret_cast<f32x4*>(win + ta.win_bytes);
  float* sb = reinterpret_cast<float*>(sw + NT * nkc * 64);
  const int lane = threadIdx.x & 63;
  const int q = lane >> 4, n = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tstride = int(gridDim.x);  // one output block (n_ob == 1) on this path
  const int wrow_bytes = ta.win_w * ta.ps;  // LDS bytes per window row

  // Window unit u (< ta.units) is 64 consecutive 16-byte pieces of window row
  // u / upr: pieces 64 (u % upr) .. + 63, piece p holding channels 4 (p % cq) ..
  // + 3 of window column p / cq (cq = cin / 4).  Wave w of W loads units w, w + W,
  // ..: slot s of a batch starting at slot s0 is unit w + W (s0 + s).  A unit is one
  // buffer load per lane from a descriptor over its image row alone (no records
  // for a row outside the image), so pieces left or right of the image read
  // zero; lanes past the row's last piece load and are not committed.
  f32x4 raw[kWinSlots];
  // The slots' unit arithmetic (row, column, descriptor) runs on the vector ALU
  // from a per-lane copy of the uniform unit index, and only the descriptor's
  // fields go back to scalar registers: the walk is uniform, but the CU's eight
  // waves share one scalar ALU, and in scalar form this walk made it the CU's
  // busiest unit.  (The copy is an asm move, so the compiler cannot fold it
  // back to scalar code.)
  auto vcopy = [](int v) {
    int r;
    asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "s"(v));
    return r;
  };
  auto win_issue = [&](int tile, int s0) {
    const int th = tile / ta.tiles_w, tw = tile - th * ta.tiles_w;
    const int cshift = (tw * kTileW - a.pw) * a.cin * 4;  // bytes; negative at the left edge
    const int64_t rstep = int64_t(a.W) * a.cin * 4;      // bytes per image row
    const int ih0 = th * kTileH - a.ph;
    const int u0 = vcopy(wave + kCtWaves * s0);
    // every slot loads (a unit past the window, or a row outside the image, has no records and reads
    // zero), so the counts of loads in flight are exact and the waits for older loads stay narrow
#pragma unroll
    for (int s = 0; s < kWinSlots; ++s) {
      const int u = u0 + kCtWaves * s;
      const int r = int(__umulhi(unsigned(u), ta.upr_magic)), c = u - r * ta.upr;
      const int ih = ih0 + r;
      const int nrec = (u < ta.units && unsigned(ih) < unsigned(a.H)) ? ta.row_bytes : 0;
      const uint64_t row = uint64_t(a.x) + uint64_t(int64_t(ih) * rstep);  // image row ih (no records outside)
      const uint32_t rlo = __builtin_amdgcn_readfirstlane(uint32_t(row));
      const uint32_t rhi = __builtin_amdgcn_readfirstlane(uint32_t(row >> 32));
      const auto rs = __builtin_amdgcn_make_buffer_rsrc(
          reinterpret_cast<void*>((uint64_t(rhi) << 32) | rlo), 0, __builtin_amdgcn_readfirstlane(nrec), 0x00020000);
      raw[s] = __builtin_bit_cast(
          f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, unsigned(16 * lane + c * 1024 + cshift), 0, 0));
    }
  };
  auto win_commit = [&](int s0) {
    const int u0 = vcopy(wave + kCtWaves * s0);
#pragma unroll
    for (int s = 0; s < kWinSlots; ++s) {
      const int u = u0 + kCtWaves * s;
      const int r = int(__umulhi(unsigned(u), ta.upr_magic)), c = u - r * ta.upr;
      const int p = 64 * c + lane;
      // window pixel p / cq at (p / cq) ps, its 4-channel group p % cq at 8 (p % cq): 8 p + 16 (p / cq);
      // a lane past the row's pieces (or a slot past the window) writes the spare 8 bytes after the
      // window instead, so the write needs no exec mask
      const int col = int(__umulhi(unsigned(p), ta.cq_magic));
      const int dst = (u < ta.units && p < ta.rp) ? r * wrow_bytes + 8 * p + 16 * col : ta.win_bytes - 16;
      half4 hv;
#pragma unroll
      for (int j = 0; j < 4; ++j) hv[j] = half_t(raw[s][j]);
      *reinterpret_cast<half4*>(win + dst) = hv;
    }
  };

  int tile = int(blockIdx.x);  // tiles < 2^31 (checked on the host)
  // the filter's first round of loads, then the first window's (or its first batch), then the conversions
  // (the grid has at most one block per tile, so every block has a first tile)
  ct_stage_filter<NT>(a.w, a.bias, nkc, sw, sb, [&]() { win_issue(tile, 0); });
  for (; tile < ta.tiles; tile += tstride) {
    const int th = tile / ta.tiles_w, tw = tile - th * ta.tiles_w;
    const int h0 = th * kTileH, w0 = tw * kTileW;
    // this tile's window into LDS: the batch in flight, and any further batches now
    win_commit(0);
    for (int s0 = kWinSlots; kCtWaves * s0 < ta.units; s0 += kWinSlots) {
      win_issue(tile, s0);
      win_commit(s0);
    }
    __syncthreads();
    // the next tile's window loads run under this tile's MFMAs
    const int next = tile + tstride;  // (tiles <= 2^30 and the grid is at most one block per CU)
    if (next < ta.tiles) win_issue(next, 0);  // (its first batch, when the window needs more than one)
    f32x4 acc[kNB][NT];
    if (wave < kMath) {  // the MFMAs
    {
      const f32x4* sb4 = reinterpret_cast<const f32x4*>(sb);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const f32x4 b = sb4[t * 4 + q];
#pragma unroll
        for (int j = 0; j < kNB; ++j) acc[j][t] = b;
      }
    }
    // lane (q, n) of N block j reads window pixel (kRows wave + j / 2 + kh, 16 (j % 2) + n + kw),
    // channels 32 kc + 8 q .. + 7, and of output tile t filter slot (t nkc + chunk) 64 +
    // cv_swz(t, lane).  Each fragment's LDS address lives in a register of its own and
    // moves by a uniform step per chunk (channels first, then taps along the row, then
    // rows), so a chunk's reads need no address arithmetic.  Two register sets
    // alternate: chunk c + 1's fragments are read into one while chunk c's MFMAs run on
    // the other, and a scheduling barrier keeps the reads ahead of those MFMAs.  Every
    // read is unconditional: past the last chunk the addresses stay on it (a re-read,
    // unused), so the waits before each MFMA group count exactly the reads in flight.
    const int kcs = a.cin / 32;
    unsigned xo[kNB], wo[NT];
    {
      const unsigned xb0 = unsigned((kRows * wave * ta.win_w + n) * ta.ps + 16 * q);
#pragma unroll
      for (int j = 0; j < kNB; ++j) xo[j] = xb0 + unsigned((j >> 1) * wrow_bytes + (j & 1) * 16 * ta.ps);
#pragma unroll
      for (int t = 0; t < NT; ++t) wo[t] = unsigned(ta.win_bytes + (t * nkc * 64 + cv_swz(t, lane)) * 16);
    }
    int kc = 0, kw = 0, cn = 0;  // the next read's channel chunk, tap column and chunk index
    auto frags = [&](half8 (&xb)[kNB], half8 (&wb)[NT]) {
#pragma unroll
      for (int j = 0; j < kNB; ++j) xb[j] = *reinterpret_cast<const half8*>(win + xo[j]);
#pragma unroll
      for (int t = 0; t < NT; ++t) wb[t] = *reinterpret_cast<const half8*>(win + wo[t]);
      if (++cn < nkc) {
        int d = 64;
        if (++kc == kcs) {
          kc = 0;
          if (++kw == a.kw) {
            kw = 0;
            d = (ta.win_w - a.kw + 1) * ta.ps - 64 * (kcs - 1);
          } else {
            d = ta.ps - 64 * (kcs - 1);
          }
        }
#pragma unroll
        for (int j = 0; j < kNB; ++j) xo[j] += unsigned(d);
#pragma unroll
        for (int t = 0; t < NT; ++t) wo[t] += 1024u;
      }
    };
    auto mma = [&](const half8 (&xb)[kNB], const half8 (&wb)[NT]) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int j = 0; j < kNB; ++j)
          acc[j][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wb[t], xb[j], acc[j][t], 0, 0, 0);
    };
    half8 xa[kNB], wa[NT], xb2[kNB], wb2[NT];
    frags(xa, wa);
    int c = 0;
    for (; c + 2 <= nkc; c += 2) {
      frags(xb2, wb2);  // chunk c + 1
      __builtin_amdgcn_sched_barrier(0);
      mma(xa, wa);      // chunk c
      frags(xa, wa);    // chunk c + 2 (a re-read of the last chunk when there is none)
      __builtin_amdgcn_sched_barrier(0);
      mma(xb2, wb2);    // chunk c + 1
    }
    if (c < nkc) mma(xa, wa);  // an odd chunk count's last chunk
    if (a.relu) {
#pragma unroll
      for (int j = 0; j < kNB; ++j)
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[j][t][e] = fmaxf(acc[j][t][e], 0.0f);
    }
    }  // the MFMAs
    if constexpr ((NT & (NT - 1)) == 0) {
      if (ta.stage_out) {
        // Each N block's outputs (16 pixels x 16 NT channels, contiguous in y) go out
        // in 1 KiB stores of consecutive lanes: the wave stages them in NT KiB of the
        // window's LDS (every wave is done reading it after this barrier), a pixel's
        // 16-byte units XORed by the pixel's low bits so that the writes (16 pixels a
        // stride apart) and the reads (one pixel's units) both spread over the banks;
        // one wave writes and reads its own slot, in order.
        __syncthreads();
        constexpr int U = 4 * NT;  // 16-byte units per pixel
        uint8_t* slot = win + wave * (1024 * NT);
        if (wave < kMath) {
#pragma unroll
          for (int j = 0; j < kNB; ++j) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
              *reinterpret_cast<f32x4*>(slot + n * (64 * NT) + 16 * ((4 * t + q) ^ (n & (U - 1)))) = acc[j][t];
            const int oh = h0 + kRows * wave + (j >> 1), pw0 = w0 + 16 * (j & 1);
#pragma unroll
            for (int k = 0; k < NT; ++k) {
              const int px = k * (16 / NT) + lane / U, u = lane % U;
              const f32x4 v = *reinterpret_cast<const f32x4*>(slot + px * (64 * NT) + 16 * (u ^ (px & (U - 1))));
              if (oh < a.H && pw0 + px < a.W)
                __builtin_nontemporal_store(
                    v, reinterpret_cast<f32x4*>(a.y + (int64_t(oh) * a.W + pw0 + px) * a.cout + 4 * u));
            }
          }
        }
        __syncthreads();  // every wave is done with this window
        continue;
      }
    }
    if (wave < kMath) {
#pragma unroll
      for (int j = 0; j < kNB; ++j) {
        const int oh = h0 + kRows * wave + (j >> 1), ow = w0 + 16 * (j & 1) + n;
        if (oh < a.H && ow < a.W) {
          float* yr = a.y + (int64_t(oh) * a.W + ow) * a.cout;
#pragma unroll
          for (int t = 0; t < NT; ++t)
            __builtin_nontemporal_store(acc[j][t], reinterpret_cast<f32x4*>(yr + 16 * t + 4 * q));
        }
      }
    }
    __syncthreads();  // every wave is done with this window
  }
}

template <bool F16, int NT, bool VEC>
const void* cv_fn() {
  return reinterpret_cast<const void*>(&conv_op_kernel<F16, NT, VEC>);
}

}  // namespace

int conv2d_check(const rdv_conv2d_desc& d, std::string* why) {
  auto bad = [&](const std::string& m) {
    *why = m;
    return RDV_ERR_INVALID;
  };
  if (d.H < 0 || d.W < 0) return bad("H and W must be >= 0");
  if (d.kh < 1 || d.kw < 1 || d.kh > 31 || d.kw > 31) return bad("kernel size must be in [1, 31]");
  if (d.precision != RDV_PREC_F16 && d.precision != RDV_PREC_F32) return bad("unknown precision code");
  if (d.w_layout != RDV_WLAYOUT_RSCK && d.w_layout != RDV_WLAYOUT_KCRS) return bad("unknown filter layout");
  if (d.cin < 1) return bad("in_channels (" + std::to_string(d.cin) + ") must be >= 1");
  if (d.cout < 1) return bad("out_channels (" + std::to_string(d.cout) + ") must be >= 1");
  if (int64_t(d.kh) * d.kw * d.cin > (int64_t(1) << 20)) return bad("kernel too large");
  if (int64_t(d.H) * d.W * std::max(d.cin, d.cout) >= (int64_t(1) << 40)) return bad("image too large");
  if (d.H > (1 << 24) || d.W > (1 << 24)) return bad("image too large");
  return RDV_OK;
}

int launch_conv2d(const rdv_conv2d_desc& d, const float* x, const float* w, const float* bias, float* y,
                  hipStream_t stream) {
  const int cstep = d.precision == RDV_PREC_F16 ? 8 : 4;
  const bool vec = d.cin % cstep == 0 && d.cout % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(y) % 16 == 0;
  const int64_t rows = int64_t(d.H) * d.W;
  if (rows == 0) return RDV_OK;
  DeviceInfo dev;
  if (int rc = device_info(&dev)) return rc;
  const bool f16 = d.precision == RDV_PREC_F16;
  const int step = f16 ? 32 : 16;
  const int esize = f16 ? 2 : 4;
  const int K = d.kh * d.kw * d.cin;
  const int Kp = (K + step - 1) / step * step;
  const int cout16 = (d.cout + 15) / 16 * 16;
  // the largest output block whose whole K fits in LDS, else 16 outputs and K passes
  int ob = std::min(kCvMaxOb, cout16);
  while (ob > 16 && int64_t(ob) * Kp * esize > kCvLdsCap) ob /= 2;
  ob = std::max(16, ob / 16 * 16);
  int kp = Kp, passes = 1;
  if (int64_t(ob) * Kp * esize > kCvLdsCap) {
    const int kmax = int(kCvLdsCap / (int64_t(ob) * esize)) / step * step;
    passes = (Kp + kmax - 1) / kmax;
    kp = ((Kp + passes - 1) / passes + step - 1) / step * step;
  }
  ConvArgs a;
  a.x = x;
  a.w = w;
  a.bias = bias;
  a.y = y;
  a.rows = rows;
  a.H = d.H;
  a.W = d.W;
  a.cin = d.cin;
  a.cout = d.cout;
  a.kh = d.kh;
  a.kw = d.kw;
  a.ph = d.kh / 2;
  a.pw = d.kw / 2;
  a.K = K;
  a.wlayout = d.w_layout;
  a.relu = d.relu ? 1 : 0;
  a.kp = kp;
  a.passes = passes;
  a.ob = ob;
  a.n_ob = (d.cout + ob - 1) / ob;
  a.w_rows = d.w_layout == RDV_WLAYOUT_RSCK && d.cout % 4 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0 ? 1 : 0;
  // spatial tiles: fp16, whole 32-channel chunks per tap, an RSCK filter of
  // 16-byte rows, one output block, and the haloed window plus the filter block in LDS
  // (and image rows whose bytes a buffer descriptor's 31-bit record count covers)
  if (f16 && vec && a.w_rows && d.cin % 32 == 0 && d.cout % 16 == 0 && passes == 1 && a.n_ob == 1 &&
      int64_t(d.W) * d.cin * 4 < (int64_t(1) << 31)) {
    const int64_t tiles = int64_t((d.H + kTileH - 1) / kTileH) * ((d.W + kTileW - 1) / kTileW);
    if (tiles > (int64_t(1) << 30)) return fail(RDV_ERR_UNSUPPORTED, "grid too large");
    const size_t filt = size_t(ob / 16) * (K / 32) * 64 * sizeof(f32x4) + size_t(ob) * sizeof(float);
    const int ti = ob / 16 - 1;  // the kernels' NT is the exact tile count
    const int64_t grid = std::min<int64_t>(tiles, dev.cu_count);
    TileArgs ta;
    ta.c = a;
    ta.c.kp = K;
    ta.win_w = kTileW + d.kw - 1;
    ta.win_h = kTileH + d.kh - 1;
    ta.ps = 2 * d.cin + 16;
    ta.win_bytes = (ta.win_w * ta.win_h * ta.ps + 15) / 16 * 16 + 16;
    ta.rp = ta.win_w * (d.cin / 4);
    ta.upr = (ta.rp + 63) / 64;
    ta.units = ta.win_h * ta.upr;
    ta.row_bytes = int(int64_t(d.W) * d.cin * 4);
    ta.cq_magic = unsigned(((uint64_t(1) << 32) + unsigned(d.cin / 4) - 1) / unsigned(d.cin / 4));
    ta.upr_magic = unsigned(((uint64_t(1) << 32) + unsigned(ta.upr) - 1) / unsigned(ta.upr));
    static const int tmath[8] = {ct_math<1>(), ct_math<2>(), ct_math<3>(), ct_math<4>(),
                                 ct_math<5>(), ct_math<6>(), ct_math<7>(), ct_math<8>()};
    ta.stage_out = ta.win_bytes >= tmath[ti] * 1024 * (ob / 16) ? 1 : 0;
    static const int tthreads[8] = {ct_threads<1>(), ct_threads<2>(), ct_threads<3>(), ct_threads<4>(),
                                    ct_threads<5>(), ct_threads<6>(), ct_threads<7>(), ct_threads<8>()};
    const size_t tlds = size_t(ta.win_bytes) + filt;
    if (tlds <= size_t(156) * 1024) {
      ta.tiles_w = (d.W + kTileW - 1) / kTileW;
      ta.tiles = int(tiles);
      static const void* const tfns[8] = {
          reinterpret_cast<const void*>(&conv_tile_kernel<1>), reinterpret_cast<const void*>(&conv_tile_kernel<2>),
          reinterpret_cast<const void*>(&conv_tile_kernel<3>), reinterpret_cast<const void*>(&conv_tile_kernel<4>),
          reinterpret_cast<const void*>(&conv_tile_kernel<5>), reinterpret_cast<const void*>(&conv_tile_kernel<6>),
          reinterpret_cast<const void*>(&conv_tile_kernel<7>), reinterpret_cast<const void*>(&conv_tile_kernel<8>)};
      static bool tattr[8] = {};
      if (!tattr[ti]) {
        RDV_HIP_TRY(hipFuncSetAttribute(tfns[ti], hipFuncAttributeMaxDynamicSharedMemorySize, 156 * 1024));
        tattr[ti] = true;
      }
      void* tparams[] = {&ta};
      RDV_HIP_TRY(hipLaunchKernel(tfns[ti], dim3(static_cast<unsigned>(grid)), dim3(tthreads[ti]), tparams, tlds, stream));
      return RDV_OK;
    }
  }
  const int64_t rows_per_task = int64_t(kCvWaves) * 16 * kCvRT;
  a.tasks = (rows + rows_per_task - 1) / rows_per_task;
  const int nt = ob / 16;
  const int ti = nt <= 2 ? 0 : nt <= 4 ? 1 : 2;
  static const void* const fns[2][2][3] = {
      {{cv_fn<false, 2, false>(), cv_fn<false, 4, false>(), cv_fn<false, 8, false>()},
       {cv_fn<false, 2, true>(), cv_fn<false, 4, true>(), cv_fn<false, 8, true>()}},
      {{cv_fn<true, 2, false>(), cv_fn<true, 4, false>(), cv_fn<true, 8, false>()},
       {cv_fn<true, 2, true>(), cv_fn<true, 4, true>(), cv_fn<true, 8, true>()}}};
  const void* fn = fns[f16][vec][ti];
  const size_t lds = size_t(nt) * (kp / step) * 64 * sizeof(f32x4) + size_t(ob) * sizeof(float);
  static bool attr_set[2][2][3] = {};
  bool& set = attr_set[f16][vec][ti];
  if (!set) {
    RDV_HIP_TRY(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    int(kCvLdsCap + kCvMaxOb * sizeof(float))));
    set = true;
  }
  int occ = 0;
  RDV_HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, kCvThreads, lds));
  occ = std::max(occ, 1);
  const int64_t slots = int64_t(dev.cu_count) * occ;
  const int64_t rwgs = std::max<int64_t>(1, std::min<int64_t>(a.tasks, (slots + a.n_ob - 1) / a.n_ob));
  const int64_t grid = rwgs * a.n_ob;
  if (grid > 0x7fffffff) return fail(RDV_ERR_UNSUPPORTED, "grid too large");
  void* params[] = {&a};
  RDV_HIP_TRY(hipLaunchKernel(fn, dim3(static_cast<unsigned>(grid)), dim3(kCvThreads), params, lds, stream));
  return RDV_OK;
}

}  // namespace rdv
