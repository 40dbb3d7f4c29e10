// D = 128 instantiations of the attention kernels (lvsa_attn_kernels.h), in a
// translation unit of their own so that the build can give them the max-ILP
// machine scheduler (-mllvm -amdgpu-sched-strategy=max-ilp).
#include "lvsa_attn_stream.h"

namespace lvsa {

int launch_d128(const AttnParams& prm, int block_q, bool bf16, hipStream_t stream) {
  if (block_q == kPPBM && prm.use_stream) {
    if (bf16) {
      hipLaunchKernelGGL((attn_fwd_stream_kernel<128, 8, __bf16>), dim3(prm.grid), dim3(kPPThreads), 0, stream,
                         prm);
    } else {
      hipLaunchKernelGGL((attn_fwd_stream_kernel<128, 8, _Float16>), dim3(prm.grid), dim3(kPPThreads), 0,
                         stream, prm);
    }
    return launch_status("lvsa_attn_fwd");
  }
  return bf16 ? launch<128, __bf16>(prm, block_q, stream) : launch<128, _Float16>(prm, block_q, stream);
}

}  // namespace lvsa
