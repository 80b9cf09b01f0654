// Thread-local error text for the C ABI and the checks that set it.
#pragma once

#include <stdarg.h>
#include <stdio.h>

#include <string>

namespace sk {

inline std::string& last_error() {
  static thread_local std::string msg;
  return msg;
}

inline int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  last_error() = buf;
  return code;
}

}  // namespace sk

#define SK_CHECK(cond, code, ...)                        \
  do {                                                   \
    if (!(cond)) return ::sk::fail((code), __VA_ARGS__); \
  } while (0)

#define SK_HIP(call)                                                                      \
  do {                                                                                    \
    const hipError_t _e = (call);                                                         \
    if (_e != hipSuccess)                                                                 \
      return ::sk::fail(SK_EHIP, "%s failed: %s", #call, hipGetErrorString(_e));          \
  } while (0)
