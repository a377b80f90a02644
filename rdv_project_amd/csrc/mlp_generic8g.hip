// The 8-tile runtime-shaped MLP kernel reading its weights from global memory
// (chains too large for LDS), compiled on its own: see mlp_generic_fwd.h.
#include "mlp_generic_fwd.h"

namespace rdv {

int launch_generic_mt8_global(const GenFwdArgs& a, int64_t blocks, hipStream_t stream) {
  return launch_generic_t<8, false>(a, blocks, 0, stream);
}

}  // namespace rdv
