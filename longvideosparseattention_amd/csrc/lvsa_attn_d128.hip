// D = 128 instantiations of the attention kernels (lvsa_attn_kernels.h), in a
// translation unit of their own so that the build can give them the max-ILP
// machine scheduler (-mllvm -amdgpu-sched-strategy=max-ilp).
#include "lvsa_attn_kernels.h"

namespace lvsa {

int launch_d128(const AttnParams& prm, int block_q, bool bf16, hipStream_t stream) {
  return bf16 ? launch<128, __bf16>(prm, block_q, stream) : launch<128, _Float16>(prm, block_q, stream);
}

}  // namespace lvsa
