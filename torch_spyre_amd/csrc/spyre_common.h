// Shared helpers of libspyre_hip: error reporting and argument checks.
#pragma once

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/spyre_hip.h"

namespace spyre_hip {

// Records the message of the last failure on this thread (spyre_last_error).
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

}  // namespace spyre_hip

#define SPYRE_REQUIRE(cond, code, ...)    \
  do {                                    \
    if (!(cond)) {                        \
      spyre_hip::set_error(__VA_ARGS__);  \
      return (code);                      \
    }                                     \
  } while (0)
