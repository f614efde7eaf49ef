// Shared helpers of the hi3d_amd HIP library: status handling, dtype tags,
// vector types and small device utilities. gfx950 (CDNA4, wave64) only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/hi3d_amd.h"

namespace hi3d {

// Last error message of the calling host thread (returned by hi3d_last_error).
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);

#define HI3D_HIP_CHECK(expr)                                                        \
  do {                                                                              \
    hipError_t e_ = (expr);                                                         \
    if (e_ != hipSuccess)                                                           \
      return ::hi3d::fail(HI3D_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

#define HI3D_LAUNCH_CHECK()                                                          \
  do {                                                                              \
    hipError_t e_ = hipGetLastError();                                              \
    if (e_ != hipSuccess)                                                           \
      return ::hi3d::fail(HI3D_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e_)); \
  } while (0)

#define HI3D_REQUIRE(cond, ...)                                                      \
  do {                                                                              \
    if (!(cond)) return ::hi3d::fail(HI3D_ERR_INVALID, __VA_ARGS__);                 \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Compute units of the current device (queried once per device).
inline int compute_units() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cached[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cached[dev] = v;
  }
  return cached[dev];
}

inline int64_t align_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

// Bump allocator over a caller-provided workspace (the library never allocates).
struct Workspace {
  char* base;
  int64_t size;
  int64_t used = 0;
  Workspace(void* p, int64_t s) : base(static_cast<char*>(p)), size(s) {}
  template <typename T>
  T* take(int64_t count) {
    used = align_up(used, 256);
    T* p = reinterpret_cast<T*>(base + used);
    used += count * static_cast<int64_t>(sizeof(T));
    return p;
  }
  bool ok() const { return used <= size; }
};

// Fill kernel (used instead of hipMemsetAsync so a caller may capture the
// library's launches in a HIP graph).
template <typename T>
__global__ void fill_kernel(T* __restrict__ p, int64_t n, T v) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (; i < n; i += stride) p[i] = v;
}

template <typename T>
inline void launch_fill(T* p, int64_t n, T v, hipStream_t s) {
  if (n <= 0) return;
  int64_t blocks = ceil_div(n, 256);
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(fill_kernel<T>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, p, n, v);
}

}  // namespace hi3d
