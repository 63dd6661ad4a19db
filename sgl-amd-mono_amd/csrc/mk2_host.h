// Host-side helpers of the C ABI: error text, argument checks, workspace carving.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#include "mk2.h"

namespace mk2 {

int set_error(int code, const char* fmt, ...);
void clear_error();

// bump allocator over the caller's workspace (256-byte aligned pieces)
struct Carver {
  char* base;
  size_t used = 0;
  explicit Carver(void* b) : base((char*)b) {}
  template <typename T>
  T* take(size_t count) {
    used = (used + 255) & ~(size_t)255;
    T* p = base ? (T*)(base + used) : nullptr;
    used += count * sizeof(T);
    return p;
  }
  size_t bytes() const { return (used + 255) & ~(size_t)255; }
};

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(MK2_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
  return MK2_OK;
}

}  // namespace mk2

#define MK2_REQUIRE(cond, ...)                               \
  do {                                                       \
    if (!(cond)) return mk2::set_error(MK2_EINVAL, __VA_ARGS__); \
  } while (0)
