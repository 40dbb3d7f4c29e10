// Shared host/device helpers of the LVSA MI355X library.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "lvsa_amd.h"

namespace lvsa {

// Thread-local last-error message (lvsa_last_error()).
void set_error(const char* fmt, ...);
void clear_error();

// Check the result of an asynchronous launch without synchronising.
inline int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return LVSA_ERR_HIP;
  }
  return LVSA_OK;
}

#define LVSA_REQUIRE(cond, code, ...) \
  do {                                \
    if (!(cond)) {                    \
      ::lvsa::set_error(__VA_ARGS__); \
      return (code);                  \
    }                                 \
  } while (0)

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Plan entry descriptor layout (documented in lvsa_amd.h).
enum : uint32_t {
  kKindNone = 0u,
  kKindTwoPart = 1u,
  kKindGeneric = 2u,
  kSrcExtra = 0x80000000u,
};

__host__ __device__ inline uint32_t make_desc(uint32_t kind, uint32_t bits, uint32_t ksplit, uint32_t qsplit) {
  return kind | (bits << 2) | (ksplit << 8) | (qsplit << 16);
}

// Smallest workspace lvsa_attn_fwd runs a call with: the text-split partials
// and the work-queue counters, without the video split's partials (which
// lvsa_attn_workspace_query adds and lvsa_attn_fwd uses when they fit).
int64_t attn_workspace_min_bytes(const lvsa_attn_args* a);

}  // namespace lvsa
