// Host-side helpers shared by the library's translation units: the
// per-thread error message and launch checking.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/voyager_hip.h"

namespace vh {

void set_error(const char* fmt, ...);

// Check the launch that was just issued; returns VH_OK or VH_ELAUNCH.
int check_launch(const char* what);

inline hipStream_t as_stream(vh_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

inline int dtype_size(int dt) {
  switch (dt) {
    case VH_BF16: case VH_F16: return 2;
    case VH_F32: return 4;
    case VH_U8: return 1;
    case VH_I64: return 8;
    default: return 0;
  }
}

inline bool is_float_dtype(int dt) { return dt == VH_BF16 || dt == VH_F32 || dt == VH_F16; }

}  // namespace vh

#define VH_REQUIRE(cond, ...)        \
  do {                               \
    if (!(cond)) {                   \
      vh::set_error(__VA_ARGS__);    \
      return VH_EINVAL;              \
    }                                \
  } while (0)
