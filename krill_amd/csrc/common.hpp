// Shared status codes and per-thread error text for libkrillhip.
#pragma once

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/libkrillhip.h"

namespace krill {

inline thread_local std::string g_last_error;

// Record a formatted message for krill_last_error() and return `code`.
inline int32_t fail(int32_t code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

inline void clear_error() { g_last_error.clear(); }

}  // namespace krill
