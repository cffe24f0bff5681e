// Error reporting shared by the library's translation units: one
// thread-local message per calling thread, read back by exl3_last_error().
#pragma once

#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <string>

namespace exl3 {

inline thread_local std::string g_last_error;

inline int set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
inline int set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return 1;
}

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error("%s: launch failed: %s", what, hipGetErrorString(e));
  return 0;
}

// Blocks of `block` threads covering `total` elements of a 1-D launch, or
// an error when that exceeds the grid limit.
inline int grid_1d(int64_t total, int block, unsigned* blocks, const char* what) {
  const int64_t b = (total + block - 1) / block;
  if (total <= 0 || b > (int64_t)INT32_MAX) return set_error("%s: batch too large", what);
  *blocks = (unsigned)b;
  return 0;
}

}  // namespace exl3
