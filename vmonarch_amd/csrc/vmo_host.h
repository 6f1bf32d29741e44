// Host-side helpers shared by the C-ABI entry points (error state, argument checks).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include "../../include/vmonarch_amd.h"

namespace vmo {

// Records a message for vmo_last_error() (thread-local) and returns `code`.
int set_error(int code, const char* fmt, ...);
void clear_error();

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Rows of a view must start on 16-byte boundaries: every stride a multiple of 8 elements.
inline bool view_ok(const vmo_view& v) {
  return v.data != nullptr && aligned16(v.data) && v.stride_b % 8 == 0 && v.stride_h % 8 == 0 &&
         v.stride_n % 8 == 0 && v.stride_n > 0;
}

inline int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(VMO_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return VMO_OK;
}

// Number of 8-XCD-aligned workgroups for `n` logical workgroups (the kernels remap block ids so
// that consecutive logical tiles share one XCD and its L2).
inline int xcd_grid(int n) { return (n + 7) / 8 * 8; }

}  // namespace vmo
