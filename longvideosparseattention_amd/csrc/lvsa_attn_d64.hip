// D = 64 instantiations of the attention kernels
// (lvsa_attn_kernels.h), in a translation unit of their own so that adding
// them leaves the compiler's code for the other head sizes unchanged.
#include "lvsa_attn_kernels.h"

namespace lvsa {

int launch_d64(const AttnParams& prm, int block_q, bool bf16, hipStream_t stream) {
  return bf16 ? launch<64, __bf16>(prm, block_q, stream) : launch<64, _Float16>(prm, block_q, stream);
}

}  // namespace lvsa
