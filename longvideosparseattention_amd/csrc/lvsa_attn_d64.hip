// D = 64 instantiations of the attention kernels
// (lvsa_attn_kernels.h, lvsa_attn_stream.h), in a translation unit of their
// own so that adding them leaves the compiler's code for the other head sizes
// unchanged.  Tiles of 384 rows run the 12-wave single-stream kernel (three
// waves per SIMD); tiles of 256 rows the 8-wave one or the ping-pong kernel.
#include "lvsa_attn_stream.h"

namespace lvsa {

int launch_d64(const AttnParams& prm, int block_q, bool bf16, hipStream_t stream) {
  if (block_q == kStream12BM) {
    if (bf16) {
      hipLaunchKernelGGL((attn_fwd_stream_kernel<64, 12, __bf16>), dim3(prm.grid), dim3(64 * 12), 0, stream, prm);
    } else {
      hipLaunchKernelGGL((attn_fwd_stream_kernel<64, 12, _Float16>), dim3(prm.grid), dim3(64 * 12), 0, stream,
                         prm);
    }
    return launch_status("lvsa_attn_fwd");
  }
  if (block_q == kPPBM && prm.use_stream && prm.dual) {
    // 4 waves of 64 rows, two work-groups per CU
    if (bf16) {
      hipLaunchKernelGGL((attn_fwd_stream_kernel<64, 4, __bf16>), dim3(prm.grid), dim3(64 * 4), 0, stream, prm);
    } else {
      hipLaunchKernelGGL((attn_fwd_stream_kernel<64, 4, _Float16>), dim3(prm.grid), dim3(64 * 4), 0, stream,
                         prm);
    }
    return launch_status("lvsa_attn_fwd");
  }
  if (block_q == kPPBM && prm.use_stream) {
    if (bf16) {
      hipLaunchKernelGGL((attn_fwd_stream_kernel<64, 8, __bf16>), dim3(prm.grid), dim3(kPPThreads), 0, stream, prm);
    } else {
      hipLaunchKernelGGL((attn_fwd_stream_kernel<64, 8, _Float16>), dim3(prm.grid), dim3(kPPThreads), 0, stream,
                         prm);
    }
    return launch_status("lvsa_attn_fwd");
  }
  return bf16 ? launch<64, __bf16>(prm, block_q, stream) : launch<64, _Float16>(prm, block_q, stream);
}

}  // namespace lvsa
