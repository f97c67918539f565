// Host-side helpers for the extern "C" entry points: thread-local error text
// and launch checking.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "vkwr_amd.h"

namespace vk {

void set_error(const char* fmt, ...);
void clear_error();

// Returns VKWR_OK, or VKWR_ERR_LAUNCH with the HIP error text recorded.
int check_launch(const char* what);

// Compute units of the current device (cached per device; 256 if the query fails).
int device_cus();

#define VK_REQUIRE(cond, ...)          \
  do {                                 \
    if (!(cond)) {                     \
      ::vk::set_error(__VA_ARGS__);    \
      return VKWR_ERR_INVALID;         \
    }                                  \
  } while (0)

}  // namespace vk
