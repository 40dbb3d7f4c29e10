// D = 96 instantiations of the ping-pong attention kernel
// (lvsa_attn_kernels.h), in a translation unit of their own: instantiated
// next to D = 64 they change the compiler's code for the D = 64 kernel.
#include "lvsa_attn_kernels.h"

namespace lvsa {

int launch_d96(const AttnParams& prm, int block_q, bool bf16, hipStream_t stream) {
  return bf16 ? launch<96, __bf16>(prm, block_q, stream) : launch<96, _Float16>(prm, block_q, stream);
}

}  // namespace lvsa
