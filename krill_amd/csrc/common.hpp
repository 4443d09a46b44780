// Shared status codes and per-thread error text for libkrillhip.
#pragma once

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <exception>
#include <new>

#include "../../include/libkrillhip.h"

namespace krill {

// Per-thread message of the last failed call: a fixed buffer, so that
// recording an error never allocates (it also reports host allocation
// failures).
inline thread_local char g_last_error[512];

// Record a formatted message for krill_last_error() and return `code`.
inline int32_t fail(int32_t code, const char *fmt, ...) noexcept {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

inline void clear_error() noexcept { g_last_error[0] = '\0'; }

// Runs the body of a C entry point: a C++ exception never crosses the C
// ABI.  A failed host allocation becomes KRILL_E_NOMEM, anything else
// KRILL_E_INVAL, each with its message.
template <class F>
inline int32_t guarded(F &&body) noexcept {
  try {
    return body();
  } catch (const std::bad_alloc &) {
    return fail(KRILL_E_NOMEM, "host memory allocation failed");
  } catch (const std::exception &e) {
    return fail(KRILL_E_INVAL, "unexpected C++ exception: %s", e.what());
  } catch (...) {
    return fail(KRILL_E_INVAL, "unexpected C++ exception");
  }
}

}  // namespace krill
