// Internal helpers shared by the libmx translation units (not part of the ABI).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <exception>
#include <sstream>
#include <string>

#include "mx.h"

namespace mx {

// Records `msg` as the thread's last error and returns `code`.
int set_error(int code, const std::string& msg);
void clear_error();

template <class... Args>
std::string cat(const Args&... args) {
  std::ostringstream os;
  (void)std::initializer_list<int>{((os << args), 0)...};
  return os.str();
}

// `stream` argument -> hipStream_t (NULL stays HIP's null stream).
hipStream_t resolve_stream(void* s);
int current_device();

// Stream-ordered scratch: freed (returned to the cache) when it goes out of
// scope; later work on the same stream is ordered after the kernels that use it.
struct Scratch {
  void* ptr = nullptr;
  Scratch() = default;
  Scratch(const Scratch&) = delete;
  Scratch& operator=(const Scratch&) = delete;
  ~Scratch() {
    if (ptr) mx_free(ptr);
  }
  int alloc(size_t bytes, hipStream_t s) {
    if (ptr) {
      mx_free(ptr);
      ptr = nullptr;
    }
    return mx_malloc(&ptr, bytes, s);
  }
  template <class T>
  T* as() const {
    return static_cast<T*>(ptr);
  }
};

// Copies a small host table to device memory through a pinned ring buffer.
// The returned device pointer is valid for work enqueued on `s` after this
// call (the block is returned to the stream-ordered cache by `holder`).
int upload(const void* host, size_t bytes, hipStream_t s, Scratch& holder);

// Number of compute units of the current device (cached).
int cu_count();

}  // namespace mx

#define MX_HIP(expr)                                                                  \
  do {                                                                                \
    hipError_t mx_e_ = (expr);                                                        \
    if (mx_e_ != hipSuccess)                                                          \
      return ::mx::set_error(MX_ERR_HIP, ::mx::cat(#expr, ": ", hipGetErrorString(mx_e_))); \
  } while (0)

#define MX_REQUIRE(cond, code, ...) \
  do {                              \
    if (!(cond)) return ::mx::set_error((code), ::mx::cat(__VA_ARGS__)); \
  } while (0)

#define MX_TRY(expr)               \
  do {                             \
    int mx_rc_ = (expr);           \
    if (mx_rc_ != MX_OK) return mx_rc_; \
  } while (0)

// Wraps an ABI body so no C++ exception crosses the C boundary.
#define MX_ABI_BEGIN \
  ::mx::clear_error(); \
  try {
#define MX_ABI_END                                                     \
  }                                                                    \
  catch (const std::exception& e) {                                    \
    return ::mx::set_error(MX_ERR_INVALID, ::mx::cat("exception: ", e.what())); \
  }                                                                    \
  catch (...) {                                                        \
    return ::mx::set_error(MX_ERR_INVALID, "unknown exception");       \
  }
