// Instantiations of the fused flash-decoding kernel for bf16 layers, 3-bit K
// and hybrid V (every V bit width, group size, head_dim and query heads per
// KV head).
#include "iq_flash.h"

namespace iq::detail {

int flash_fused_launch_bf_vh_k3(const FusedArgs& a, int vbits, int group, int D, int nrep, bool norm, int* grid,
                                hipStream_t stream, bool launch) {
  return fused_launch_kb<3, true, true>(a, vbits, group, D, nrep, norm, grid, stream, launch);
}

}  // namespace iq::detail
