// The 8-tile runtime-shaped MLP kernel with its weights in LDS (chains with a
// layer wider than 128), compiled on its own: see mlp_generic_fwd.h.
#include "mlp_generic_fwd.h"

namespace rdv {

int launch_generic_mt8_lds(const GenFwdArgs& a, int64_t blocks, size_t lds, hipStream_t stream) {
  return launch_generic_t<8, true>(a, blocks, lds, stream);
}

}  // namespace rdv
