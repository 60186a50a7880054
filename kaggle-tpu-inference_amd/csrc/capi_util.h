// Error plumbing shared by every extern "C" entry point of libg4mi.
//
// Entry points never throw across the ABI: they return 0 on success, a
// negative G4MI_E* code for a rejected argument, or the positive hipError_t of
// a failed launch.  The message of the last failure on the calling thread is
// kept for g4mi_last_error_string().
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/g4mi.h"

namespace g4mi {

void set_error(const char* fmt, ...);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Checks the launch that was just enqueued.
inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return (int)e;
  }
  return 0;
}

}  // namespace g4mi

#define G4MI_REQUIRE(cond, code, ...)  \
  do {                                 \
    if (!(cond)) {                     \
      ::g4mi::set_error(__VA_ARGS__);  \
      return (code);                   \
    }                                  \
  } while (0)
