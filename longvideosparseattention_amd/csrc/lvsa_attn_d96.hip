// D = 96 instantiations of the attention kernels (lvsa_attn_kernels.h,
// lvsa_attn_stream.h), in a translation unit of their own: instantiated next
// to D = 64 they change the compiler's code for the D = 64 kernel.  Both lay
// D = 96 rows out on the D = 128 LDS pitch.
#include "lvsa_attn_stream.h"

namespace lvsa {

int launch_d96(const AttnParams& prm, int block_q, bool bf16, hipStream_t stream) {
  if (block_q == kPPBM && prm.use_stream) {
    if (bf16) {
      hipLaunchKernelGGL((attn_fwd_stream_kernel<96, 8, __bf16>), dim3(prm.grid), dim3(kPPThreads), 0, stream, prm);
    } else {
      hipLaunchKernelGGL((attn_fwd_stream_kernel<96, 8, _Float16>), dim3(prm.grid), dim3(kPPThreads), 0, stream,
                         prm);
    }
    return launch_status("lvsa_attn_fwd");
  }
  return bf16 ? launch<96, __bf16>(prm, block_q, stream) : launch<96, _Float16>(prm, block_q, stream);
}

}  // namespace lvsa
