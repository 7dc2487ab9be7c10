// Instantiations of the column-slice attn.V kernel for 4-bit V (every group
// size, head_dim and query heads per KV head; plain and hybrid stores).
#include "iq_av_cols.h"

namespace iq::detail {

int av_cols_launch_k4(const void* args, int group, int D, int nrep, bool hybrid, hipStream_t stream) {
  return av_cols_launch_vb<4>(*static_cast<const AVCArgs*>(args), group, D, nrep, hybrid, stream);
}

}  // namespace iq::detail
