// Host-side plumbing shared by the C-ABI entry points: error strings, argument
// checks and launch-shape helpers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <algorithm>

#include "moe_fp8.h"

namespace moe {

void set_error(const char* fn, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// K splits for the router logits GEMM: aim for >= 512 workgroups, each split
// at least 256 columns of H.
inline int router_logits_splits(int T, int H, int E) {
  long base = (long)((T + 63) / 64) * ((E + 63) / 64);
  long ks = (512 + base - 1) / base;
  long kmax = std::max(1, H / 256);
  return (int)std::max(1L, std::min(ks, kmax));
}

}  // namespace moe

#define MOE_API_BEGIN(name)   \
  const char* _moe_fn = name; \
  moe::clear_error();

#define MOE_CHECK_ARG(cond, ...)            \
  do {                                      \
    if (!(cond)) {                          \
      moe::set_error(_moe_fn, __VA_ARGS__); \
      return MOE_ERR_ARG;                   \
    }                                       \
  } while (0)

#define MOE_CHECK_SUPPORTED(cond, ...)      \
  do {                                      \
    if (!(cond)) {                          \
      moe::set_error(_moe_fn, __VA_ARGS__); \
      return MOE_ERR_UNSUPPORTED;           \
    }                                       \
  } while (0)

#define MOE_CHECK_HIP(expr)                                                              \
  do {                                                                                   \
    hipError_t _e = (expr);                                                              \
    if (_e != hipSuccess) {                                                              \
      moe::set_error(_moe_fn, "%s failed: %s", #expr, hipGetErrorString(_e));            \
      return MOE_ERR_HIP;                                                                \
    }                                                                                    \
  } while (0)

#define MOE_API_END()                                                                    \
  do {                                                                                   \
    hipError_t _e = hipGetLastError();                                                   \
    if (_e != hipSuccess) {                                                              \
      moe::set_error(_moe_fn, "kernel launch failed: %s", hipGetErrorString(_e));        \
      return MOE_ERR_HIP;                                                                \
    }                                                                                    \
    return MOE_OK;                                                                       \
  } while (0)
