// D = 192 instantiations of the attention kernels: the single-stream loop
// in its dual-wide map (256-row tiles) and its wide map (128-row tiles)
// (lvsa_attn_stream.h), and the 4-wave kernel (lvsa_attn_kernels.h) for
// geometries the loop does not take, in a translation unit of their own so
// that adding them leaves the compiler's code for the other head sizes
// unchanged.
#include "lvsa_attn_stream.h"

namespace lvsa {

int launch_d192(const AttnParams& prm, int block_q, bool bf16, hipStream_t stream) {
  if (block_q == kPPBM) {
    // the dual-wide map: 4 waves of 64 rows (one wave per SIMD), 256-row tiles
    if (bf16) {
      hipLaunchKernelGGL((attn_fwd_stream_kernel<192, 4, __bf16, true>), dim3(prm.grid), dim3(256), 0, stream, prm);
    } else {
      hipLaunchKernelGGL((attn_fwd_stream_kernel<192, 4, _Float16, true>), dim3(prm.grid), dim3(256), 0, stream,
                         prm);
    }
    return launch_status("lvsa_attn_fwd");
  }
  if (block_q == kBM && prm.use_stream) {
    // the single-stream loop, wide map: 4 waves (one per SIMD), 128-row tiles
    if (bf16) {
      hipLaunchKernelGGL((attn_fwd_stream_kernel<192, 4, __bf16>), dim3(prm.grid), dim3(256), 0, stream, prm);
    } else {
      hipLaunchKernelGGL((attn_fwd_stream_kernel<192, 4, _Float16>), dim3(prm.grid), dim3(256), 0, stream, prm);
    }
    return launch_status("lvsa_attn_fwd");
  }
  return bf16 ? launch<192, __bf16>(prm, block_q, stream) : launch<192, _Float16>(prm, block_q, stream);
}

}  // namespace lvsa
