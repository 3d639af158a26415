// Errors and small helpers shared by the HIP kernel layer. Inside the library an error is an exception
// (xtg::hip::Error, like xtg::Error in engine/include/xtg/common.h:11-16); the C ABI turns it into rc + message.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>

namespace xtg::hip {

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

[[noreturn]] inline void fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
inline void fail(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  throw Error(buf);
}

inline std::string strf(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
inline std::string strf(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return buf;
}

}  // namespace xtg::hip

#define XTG_CHECK(cond, ...)                  \
  do {                                        \
    if (!(cond)) ::xtg::hip::fail(__VA_ARGS__); \
  } while (0)

namespace xtg::hip {
// A kernel that needs more than the default 64 KiB of dynamic LDS (gfx950 has 160 KiB per CU): raise its limit
// once (defined in attention.hip).
void allow_lds(const void* fn, size_t lds);
}  // namespace xtg::hip

#define HIP_CHECK(expr)                                                                        \
  do {                                                                                         \
    hipError_t e_ = (expr);                                                                    \
    if (e_ != hipSuccess) ::xtg::hip::fail("%s failed: %s", #expr, hipGetErrorString(e_)); \
  } while (0)
