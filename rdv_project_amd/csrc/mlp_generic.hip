// Runtime-shaped fused fp16 MLP forward: host-side dispatch of the kernels in
// mlp_generic_fwd.h (which chains they serve, the kernel name, the launch).
#include "mlp_generic_fwd.h"

namespace rdv {

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
    default: return use_lds ? launch_generic_mt8_lds(a, blocks, size_t(lds), stream)
                            : launch_generic_mt8_global(a, blocks, stream);
  }
}

}  // namespace rdv
