// D = 256 instantiations of the 4-wave attention kernel
// (lvsa_attn_kernels.h), in a translation unit of their own so that adding
// them leaves the compiler's code for the other head sizes unchanged.
#include "lvsa_attn_kernels.h"

namespace lvsa {

int launch_d256(const AttnParams& prm, int block_q, bool bf16, hipStream_t stream) {
  return bf16 ? launch<256, __bf16>(prm, block_q, stream) : launch<256, _Float16>(prm, block_q, stream);
}

}  // namespace lvsa
