// lvsa_attn_fwd_noalloc: lvsa_attn_fwd with its scratch (the work-queue
// counters and the text-split partials) in a static per-GPU device array, for
// callers that cannot allocate.
//
// The array is the only device object of this translation unit, so it sits in
// a code object of its own: the runtime places it on a GPU when this entry
// point first asks for its address there, not when the attention kernels of
// the other units are loaded.
#include "lvsa_common.h"

#include <mutex>

using namespace lvsa;

namespace {

// Scratch of lvsa_attn_fwd_noalloc: one array per GPU, held until the process
// ends.  In host code `scratch` only names the symbol; its device address
// comes from hipGetSymbolAddress, once per device.
__device__ __align__(256) char scratch[LVSA_NOALLOC_SCRATCH_BYTES];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch (set up on its first call).
int scratch_of_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  LVSA_REQUIRE(e == hipSuccess, LVSA_ERR_HIP, "lvsa_attn_fwd_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  LVSA_REQUIRE(dev >= 0 && dev < kMaxDevices, LVSA_ERR_UNSUPPORTED, "lvsa_attn_fwd_noalloc: device %d", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    LVSA_REQUIRE(e == hipSuccess && ptr != nullptr, LVSA_ERR_HIP,
                 "lvsa_attn_fwd_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return LVSA_OK;
}

}  // namespace

extern "C" int lvsa_attn_fwd_noalloc(const lvsa_attn_args* a, hipStream_t stream) {
  clear_error();
  LVSA_REQUIRE(a != nullptr, LVSA_ERR_INVALID_ARG, "lvsa_attn_fwd_noalloc: null args");
  int64_t need = 0;
  int rc = lvsa_attn_workspace_query(a, &need);   // validates the arguments
  if (rc != LVSA_OK) return rc;
  // the scratch must hold the text-tile split and the queue counters; the
  // video split's partials are used when they fit as well
  need = attn_workspace_min_bytes(a);
  LVSA_REQUIRE(need <= (int64_t)LVSA_NOALLOC_SCRATCH_BYTES, LVSA_ERR_CAPACITY,
               "lvsa_attn_fwd_noalloc: the text-tile split needs %lld bytes of scratch, more than the static "
               "%lld (LVSA_NOALLOC_SCRATCH_BYTES); call lvsa_attn_fwd with a workspace instead",
               (long long)need, (long long)LVSA_NOALLOC_SCRATCH_BYTES);
  lvsa_attn_args b = *a;
  b.workspace = nullptr;
  b.workspace_bytes = 0;
  if (need > 0) {
    rc = scratch_of_current_device(&b.workspace);
    if (rc != LVSA_OK) return rc;
    b.workspace_bytes = LVSA_NOALLOC_SCRATCH_BYTES;
  }
  return lvsa_attn_fwd(&b, stream);
}
