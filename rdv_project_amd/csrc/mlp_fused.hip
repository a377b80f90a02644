// Fused fp16 matrix-core MLP: the whole layer chain evaluated per wave, weights
// resident in LDS for the life of the block, activations passed from layer to
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
// Work decomposition: one block per CU; each wave evaluates two 32-point tiles
// (two MFMA N blocks) at a time, claiming them dynamically (see the kernels).
#include "mlp_core.h"

namespace rdv {

struct FusedArgs {
  const float* x;
  float* y;
  const uint8_t* packed;  // the packed block (DIRECT kernels: unused)
  DirectWeights dw;       // the layers' fp32 parameters (DIRECT kernels)
  int64_t nrows;          // rows evaluated by this launch (starting at x / y)
  int act[RDV_MLP_MAX_LAYERS];
  MlpLayout lay;
};

// Work decomposition.  One 512-thread block (8 waves, 2 per SIMD) per CU owns a
// contiguous range of 64-row pair tiles; its waves claim them one at a time
// from an LDS counter (wave w starts on pair tile w), so the waves of a SIMD
// finish together.  Each wave evaluates a pair tile as two 32-point tiles
// staggered by half a layer (run_pair, mlp_core.h): the fp32 -> fp16 hand-off
// of one tile is interleaved with the MFMAs of the other, so VALU and matrix
// work overlap within the wave.
//  - Weights: the block copies the packed A fragments into LDS once (2048
//    waves each pulling the same 26 KiB straight from L2 serialised on a few hot
//    lines for ~3 us); each wave then reads its first 26 fragments into
//    registers, and every MFMA on a later one reads its fragment with one
//    conflict-free ds_read_b128.
//  - Input: at the top of an iteration a wave claims its next pair tile and
//    DMAs its 64 rows from HBM straight into a wave-private LDS buffer
//    (global_load_lds_dword, one per input column: lane l's row lands at
//    [d][l]), double-buffered, so no registers hold input in flight; the next
//    iteration waits for it (s_waitcnt vmcnt(0)) a whole iteration later, when
//    it has long arrived.  No barrier is needed after start-up.  The first
//    tile's DMA is issued before the weight staging, so its latency overlaps it.
//  - Output: each pair tile's stores are issued one iteration late, before the
//    next DMA, so that wait (loads and stores retire in order on gfx9) never
//    covers a store younger than an iteration.
constexpr int kWaves2 = 8;
constexpr int kThreads2 = 64 * kWaves2;

//  - DIRECT: the block builds its LDS fragments from the layers' fp32 buffers
//    (stage_net_weights_direct) instead of copying a packed block, so a caller
//    holding only nn.Linear-layout parameters needs no separate pack launch.
template <class N, bool RELU, int HEAD_ACT, bool DIRECT = false>
__global__ __launch_bounds__(kThreads2, 1) void mlp_fused_f16_kernel(FusedArgs a) {
  constexpr int D = N::kIn;
  constexpr int LL = N::kL - 1;
  constexpr int MTO = N::mt(LL);
  // One LDS block carved by hand, the input tiles first: their LDS-DMA target
  // (M0) must stay below 64 KiB, and the DIRECT staging area makes the block
  // larger than that (separate __shared__ arrays are placed by the compiler).
  constexpr int kSxBytes = kWaves2 * 2 * D * 64 * 4;
  constexpr int kSwBytes = N::kFrags * 64 * 16;
  constexpr int kSbBytes = (N::kBias * 4 + 15) / 16 * 16;
  constexpr int kSstBytes = DIRECT ? DirectStage<N, kThreads2>::kFloats * 4 : 0;
  static_assert(kSxBytes <= 65536, "the input tiles' DMA addresses must be below 64 KiB");
  __shared__ __attribute__((aligned(16))) uint8_t lds[kSxBytes + kSwBytes + kSbBytes + kSstBytes + 16];
  auto& sx = *reinterpret_cast<float (*)[kWaves2][2][D * 64]>(lds);  // each wave's input pair tiles, [d][row]
  half8* const sw = reinterpret_cast<half8*>(lds + kSxBytes);
  float* const sb = reinterpret_cast<float*>(lds + kSxBytes + kSwBytes);
  float* const sst = reinterpret_cast<float*>(lds + kSxBytes + kSwBytes + kSbBytes);  // DIRECT: fp32 weight staging
  int& s_next = *reinterpret_cast<int*>(lds + kSxBytes + kSwBytes + kSbBytes + kSstBytes);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int h = lane >> 5, col = lane & 31;

  const int64_t ntiles = (a.nrows + 63) >> 6;  // 64-row pair tiles
  const int64_t per_block = (ntiles + gridDim.x - 1) / gridDim.x;
  const int64_t t_begin = int64_t(blockIdx.x) * per_block;
  const int64_t t_end = t_begin + per_block < ntiles ? t_begin + per_block : ntiles;
  const int nt = int(t_end > t_begin ? t_end - t_begin : 0);
  bool has_bias = false;
  if constexpr (!DIRECT) has_bias = packed_has_bias(a.packed);

  // DMA of pair tile lt (64 rows, lane l -> row l, clamped to the last row) into buffer `buf`
  const int64_t last = a.nrows - 1;
  auto dma_tile = [&](int lt, int buf) {
    int64_t row = (t_begin + (lt < nt ? lt : 0)) * 64 + lane;
    row = row < last ? row : last;
    const float* src = a.x + row * D;
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const uint32_t dst = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(&sx[wave][buf][d * 64]));
      uint32_t saved;
      asm volatile(
          "s_mov_b32 %0, m0\n\t"
          "s_mov_b32 m0, %2\n\t"
          "s_nop 0\n\t"
          "global_load_lds_dword %1, off\n\t"
          "s_mov_b32 m0, %0"
          : "=&s"(saved)
          : "v"(src + d), "s"(__builtin_amdgcn_readfirstlane(dst))
          : "memory");
    }
  };
  int cur = wave;
  dma_tile(cur, 0);

  if constexpr (DIRECT) {
    const bool nz = stage_net_weights_direct<N, kThreads2>(a.dw, a.lay, sb, sw, sst);
    if (threadIdx.x == 0) s_next = kWaves2;
    has_bias = __syncthreads_or(nz ? 1 : 0) != 0;
  } else {
    stage_net_weights<N, kThreads2>(a.packed, a.lay, sb, sw);
    if (threadIdx.x == 0) s_next = kWaves2;
    __syncthreads();
  }

  auto claim = [&]() {
    int t = 0;
    if (lane == 0) t = atomicAdd(&s_next, 1);
    return __builtin_amdgcn_readfirstlane(t);
  };

  // The first 26 A fragments (every one of C2's chain) in registers, read from
  // LDS once: the MFMAs on them leave the LDS to the rest (LDS reads and MFMAs
  // of a CU contend).  26 keeps every instantiation's registers within a half
  // SIMD (at most 256 VGPRs, no spills); C2: 22.9 -> 22.3 us per call.  The
  // DIRECT kernels keep the hidden layers' first 16 (their staging needs more
  // registers; 24.8 -> 24.4 us, and 25.0 us with all 26).
  constexpr int RH0 = N::kL > 2 ? N::frag_base(1) : 0;
  constexpr int RHN = N::kL > 2 ? N::frag_base(N::kL - 1) - RH0 : 0;
  constexpr int RF0 = DIRECT ? RH0 : 0;
  constexpr int RN = DIRECT ? (RHN < 16 ? RHN : 16) : (N::kFrags < 26 ? N::kFrags : 26);
  RegLdsWeights<RF0, RN> wr;
#pragma unroll
  for (int i = 0; i < RN; ++i) wr.r[i] = sw[(RF0 + i) * 64 + lane];

  f32x4 po[2][MTO][4];
  int64_t prow = -1;
  int buf = 0;
  while (cur < nt) {
    const int nxt = claim();
    // this tile's DMA (and everything older: the stores of two iterations ago) has landed
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    float pA[D], pB[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
      pA[d] = sx[wave][buf][d * 64 + col];
      pB[d] = sx[wave][buf][d * 64 + 32 + col];
    }
    // the previous pair tile's stores, then the next tile's DMA
    if (prow >= 0) {
      if (prow < a.nrows) store_head<N>(a.y + prow * N::kOut, po[0], h);
      if (prow + 32 < a.nrows) store_head<N>(a.y + (prow + 32) * N::kOut, po[1], h);
    }
    dma_tile(nxt, buf ^ 1);
    f32x16 accA[N::kMaxMT], accB[N::kMaxMT];
    half8 bA[N::kMaxKC], bB[N::kMaxKC];
    RegLdsWeights<RF0, RN> ws = wr;
    ws.sw = sw + opaque_zero();
    ws.lane = lane;
    build_input<N>(pA, h, bA);
    if (has_bias) {
      run_pair<N, 0, RELU, true>(ws, pB, h, bA, bB, accA, accB, sb + opaque_zero());
    } else {
      run_pair<N, 0, RELU, false>(ws, pB, h, bA, bB, accA, accB, sb);
    }
#pragma unroll
    for (int t = 0; t < MTO; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          po[0][t][q][jj] = head_act<HEAD_ACT>(32 * t + 8 * q + 4 * h + jj, accA[t][4 * q + jj]);
          po[1][t][q][jj] = head_act<HEAD_ACT>(32 * t + 8 * q + 4 * h + jj, accB[t][4 * q + jj]);
        }
    prow = (t_begin + cur) * 64 + col;
    cur = nxt;
    buf ^= 1;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no DMA outstanding at exit
  if (prow >= 0) {
    if (prow < a.nrows) store_head<N>(a.y + prow * N::kOut, po[0], h);
    if (prow + 32 < a.nrows) store_head<N>(a.y + (prow + 32) * N::kOut, po[1], h);
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

template <class N, bool RELU, int HEAD_ACT, bool DIRECT = false>
int launch_fused(const FusedArgs& a, int64_t nrows, hipStream_t stream) {
  if (nrows <= 0) return RDV_OK;
  DeviceInfo di;
  int rc = device_info(&di);
  if (rc != RDV_OK) return rc;
  // one block per CU; never more waves than pair tiles
  int64_t blocks = di.cu_count;
  const int64_t need = ((nrows + 63) / 64 + kWaves2 - 1) / kWaves2;
  if (need < blocks) blocks = need;
  mlp_fused_f16_kernel<N, RELU, HEAD_ACT, DIRECT><<<dim3(unsigned(blocks)), dim3(kThreads2), 0, stream>>>(a);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

struct FusedEntry {
  int enc, in, oct, out, L, kc0, hidden_act, head_act;
  int mt[RDV_MLP_MAX_LAYERS];
  FusedLauncher fn;         // packed parameters
  FusedLauncher fn_direct;  // the layers' fp32 parameters
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
  e.fn_direct = &launch_fused<N, RELU, HEAD_ACT, true>;
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

// Can the DIRECT kernel of `e` read the chain's parameters?  Its staging copies
// whole rows of the later layers: every hidden width must be a whole number of
// 32-row tiles (the instantiated widths; a narrower layer sharing a tile count
// takes the packed path).  Layer 0's rows hold at least the encoded features
// (check_mlp ensures it).
bool direct_fused_ok(const FusedEntry* e, const rdv_mlp_desc& d) {
  if (e == nullptr) return false;
  for (int i = 1; i < d.n_layers; ++i)
    if (d.dims[i] != 32 * e->mt[i - 1]) return false;
  return true;
}

int launch_fused_entry(const FusedEntry* e, const rdv_mlp_desc& d, const MlpLayout& lay, const void* packed,
                       const float* x, float* y, int64_t nrows, hipStream_t stream) {
  FusedArgs a = {};
  a.x = x;
  a.y = y;
  a.packed = static_cast<const uint8_t*>(packed);
  a.nrows = nrows;
  for (int i = 0; i < RDV_MLP_MAX_LAYERS; ++i) a.act[i] = i < d.n_layers ? d.act[i] : 0;
  a.lay = lay;
  return e->fn(a, nrows, stream);
}

int launch_fused_entry_direct(const FusedEntry* e, const rdv_mlp_desc& d, const MlpLayout& lay,
                              const DirectWeights& dw, const float* x, float* y, int64_t nrows, hipStream_t stream) {
  FusedArgs a = {};
  a.x = x;
  a.y = y;
  a.packed = nullptr;
  a.dw = dw;
  a.nrows = nrows;
  for (int i = 0; i < RDV_MLP_MAX_LAYERS; ++i) a.act[i] = i < d.n_layers ? d.act[i] : 0;
  a.lay = lay;
  return e->fn_direct(a, nrows, stream);
}

}  // namespace rdv
