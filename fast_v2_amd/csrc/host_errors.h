// Host-side error plumbing shared by the C-ABI entry points (no HIP dependency, so the
// host-only planning code can be built and sanitized with the host compiler alone).
#pragma once

namespace fdllm {
void set_last_error(const char* fmt, ...);
int dtype_size(int dtype);  // bytes per element of an FDLLM_DTYPE_*, 0 if unknown
}  // namespace fdllm

#define FDLLM_CHECK_ARG(cond, ...)          \
  do {                                      \
    if (!(cond)) {                          \
      ::fdllm::set_last_error(__VA_ARGS__); \
      return FDLLM_ERR_INVALID_ARGUMENT;    \
    }                                       \
  } while (0)
