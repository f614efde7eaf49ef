// Sorted unique values of int64 keys with the inverse map and run lengths, on the GPU,
// and the row <-> key packing that lets integer rows use it. Replaces the reference's
// MLX argsort + run marks + scatter (src/hi3d_mac/fast_unique.py:25-91), which mesh
// extraction calls on tens of millions of cube-corner and edge rows.
//
// One radix sort of (key, position) pairs over the key bits that can differ, a run-head
// flag per sorted element, an inclusive scan of the flags (run number + 1), then one pass
// that scatters the inverse map (inverse[position] = run), the run's value and its first
// sorted index; counts are differences of first indices. Results equal
// np.unique(keys, return_inverse=True, return_counts=True) bit for bit.

#include <algorithm>
#include <type_traits>

#include "common.h"
#include "radix.h"

namespace hi3d {
namespace {

constexpr unsigned long long kSignFlip = 0x8000000000000000ull;
constexpr int kMaxRowWidth = 8;

// Sort keys: signed keys with the sign bit flipped order like unsigned ones; keys known
// to lie in [0, 2^bits) are sorted as they are (as 32-bit keys when bits <= 32).
template <typename K>
__global__ void unique_prep_kernel(const int64_t* __restrict__ keys, int64_t n, unsigned long long flip,
                                   K* __restrict__ sk, int32_t* __restrict__ pos) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  sk[i] = static_cast<K>(static_cast<unsigned long long>(keys[i]) ^ flip);
  pos[i] = static_cast<int32_t>(i);
}

template <typename K>
__global__ void unique_heads_kernel(const K* __restrict__ sk, int64_t n, int32_t* __restrict__ head) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  head[i] = (i == 0 || sk[i] != sk[i - 1]) ? 1 : 0;
}

// run[i] = number of runs up to and including element i (so run[i] - 1 is its run)
template <typename K>
__global__ void unique_scatter_kernel(const K* __restrict__ sk, const int32_t* __restrict__ pos,
                                      const int32_t* __restrict__ head, const int32_t* __restrict__ run, int64_t n,
                                      unsigned long long flip, int64_t* __restrict__ uniq,
                                      int64_t* __restrict__ inverse, int32_t* __restrict__ first,
                                      int64_t* __restrict__ n_unique) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int32_t r = run[i] - 1;
  inverse[pos[i]] = r;
  if (head[i]) {
    uniq[r] = static_cast<int64_t>(static_cast<unsigned long long>(sk[i]) ^ flip);
    first[r] = static_cast<int32_t>(i);
  }
  if (i == n - 1) n_unique[0] = r + 1;
}

__global__ void unique_counts_kernel(const int32_t* __restrict__ first, const int32_t* __restrict__ run, int64_t n,
                                     int64_t* __restrict__ counts) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t u = run[n - 1];
  if (r >= u) return;
  const int64_t end = r + 1 < u ? first[r + 1] : n;
  counts[r] = end - first[r];
}

template <typename T>
__global__ void pack_rows_kernel(const T* __restrict__ rows, int64_t n, int d, const int64_t* __restrict__ lo,
                                 const int64_t* __restrict__ extent, int64_t* __restrict__ keys) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int64_t key = 0;
  for (int j = 0; j < d; ++j) key = key * extent[j] + (static_cast<int64_t>(rows[i * d + j]) - lo[j]);
  keys[i] = key;
}

template <typename T>
__global__ void unpack_rows_kernel(const int64_t* __restrict__ keys, const int64_t* __restrict__ count, int d,
                                   const int64_t* __restrict__ lo, const int64_t* __restrict__ extent,
                                   T* __restrict__ rows) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= count[0]) return;
  int64_t rem = keys[i];
  for (int j = d - 1; j > 0; --j) {
    rows[i * d + j] = static_cast<T>(rem % extent[j] + lo[j]);
    rem /= extent[j];
  }
  rows[i * d] = static_cast<T>(rem + lo[0]);
}

// Column minima and maxima of rows [n, d]: grid-stride partials per thread, a wave
// reduction, then one 64-bit atomic min and max per column per wave (order-independent,
// so the result is deterministic).
template <typename T>
__global__ void row_bounds_kernel(const T* __restrict__ rows, int64_t n, int d, int64_t* __restrict__ lo,
                                  int64_t* __restrict__ hi) {
  int64_t mn[kMaxRowWidth], mx[kMaxRowWidth];
#pragma unroll
  for (int j = 0; j < kMaxRowWidth; ++j) {
    mn[j] = INT64_MAX;
    mx[j] = INT64_MIN;
  }
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
#pragma unroll
    for (int j = 0; j < kMaxRowWidth; ++j) {
      if (j < d) {
        const int64_t v = static_cast<int64_t>(rows[i * d + j]);
        mn[j] = v < mn[j] ? v : mn[j];
        mx[j] = v > mx[j] ? v : mx[j];
      }
    }
  }
#pragma unroll
  for (int j = 0; j < kMaxRowWidth; ++j) {
    if (j >= d) break;
    int64_t a = mn[j], b = mx[j];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      const int64_t oa = __shfl_xor(a, m), ob = __shfl_xor(b, m);
      a = oa < a ? oa : a;
      b = ob > b ? ob : b;
    }
    if ((threadIdx.x & 63) == 0) {
      atomicMin(reinterpret_cast<long long*>(lo + j), static_cast<long long>(a));
      atomicMax(reinterpret_cast<long long*>(hi + j), static_cast<long long>(b));
    }
  }
}

}  // namespace
}  // namespace hi3d

using namespace hi3d;

extern "C" int hi3d_unique_keys_workspace(int64_t n, int64_t* bytes) {
  HI3D_REQUIRE(bytes != nullptr, "bytes_host is NULL");
  HI3D_REQUIRE(n >= 0 && n < (int64_t(1) << 31) - 1, "n out of range: %lld", static_cast<long long>(n));
  const int64_t m = std::max<int64_t>(n, 1);
  *bytes = 2 * align_up(m * 8, 256) + 5 * align_up(m * 4, 256) + radix::temp_bytes(m) + 256;
  return HI3D_OK;
}

extern "C" int hi3d_unique_keys(const int64_t* keys, int64_t n, int32_t key_bits, void* workspace,
                                int64_t workspace_bytes, int64_t* uniq, int64_t* inverse, int64_t* counts,
                                int64_t* n_unique, void* stream_) {
  hipStream_t stream = as_stream(stream_);
  int64_t need = 0;
  int rc = hi3d_unique_keys_workspace(n, &need);
  if (rc != HI3D_OK) return rc;
  HI3D_REQUIRE(key_bits >= 0 && key_bits <= 63, "key_bits must be 0 (any int64) or 1..63, got %d", key_bits);
  HI3D_REQUIRE(n_unique != nullptr, "null pointer argument");
  if (n == 0) {
    hipLaunchKernelGGL(fill_kernel<int64_t>, dim3(1), dim3(64), 0, stream, n_unique, int64_t(1), int64_t(0));
    HI3D_LAUNCH_CHECK();
    return HI3D_OK;
  }
  HI3D_REQUIRE(keys && workspace && uniq && inverse, "null pointer argument");
  HI3D_REQUIRE(workspace_bytes >= need, "workspace too small");
  Workspace ws(workspace, workspace_bytes);
  auto* k0 = ws.take<unsigned long long>(n);
  auto* k1 = ws.take<unsigned long long>(n);
  auto* p0 = ws.take<int32_t>(n);
  auto* p1 = ws.take<int32_t>(n);
  auto* head = ws.take<int32_t>(n);
  auto* run = ws.take<int32_t>(n);
  auto* first = ws.take<int32_t>(n);
  const int64_t temp_bytes = radix::temp_bytes(n);
  void* temp = ws.take<char>(temp_bytes);
  const unsigned blocks = static_cast<unsigned>(ceil_div(n, 256));
  // keys within [0, 2^key_bits) sort on those bits as they are; any int64 sorts on all
  // 64 bits with the sign bit flipped
  const unsigned long long flip = key_bits == 0 ? kSignFlip : 0ull;
  const int end_bit = key_bits == 0 ? 64 : key_bits;
  // keys that fit 32 bits sort as 32-bit keys (a third fewer bytes per pass)
  auto sorted_runs = [&](auto* ka, auto* kalt) -> int {
    using K = std::remove_pointer_t<decltype(ka)>;
    hipLaunchKernelGGL(unique_prep_kernel<K>, dim3(blocks), dim3(256), 0, stream, keys, n, flip, ka, p0);
    int32_t* pa = p0;
    int32_t* palt = p1;
    HI3D_HIP_CHECK(radix::sort_pairs(temp, temp_bytes, ka, kalt, pa, palt, n, 0, end_bit, stream));
    hipLaunchKernelGGL(unique_heads_kernel<K>, dim3(blocks), dim3(256), 0, stream, ka, n, head);
    HI3D_HIP_CHECK(radix::scan(temp, temp_bytes, head, run, n, true, stream));
    hipLaunchKernelGGL(unique_scatter_kernel<K>, dim3(blocks), dim3(256), 0, stream, ka, pa, head, run, n, flip,
                       uniq, inverse, first, n_unique);
    return HI3D_OK;
  };
  rc = end_bit <= 32 ? sorted_runs(reinterpret_cast<uint32_t*>(k0), reinterpret_cast<uint32_t*>(k1))
                     : sorted_runs(k0, k1);
  if (rc != HI3D_OK) return rc;
  if (counts)
    hipLaunchKernelGGL(unique_counts_kernel, dim3(blocks), dim3(256), 0, stream, first, run, n, counts);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

extern "C" int hi3d_pack_rows(const void* rows, int32_t dtype, int64_t n, int32_t d, const int64_t* lo,
                              const int64_t* extent, int64_t* keys, void* stream_) {
  HI3D_REQUIRE(dtype == HI3D_I32 || dtype == HI3D_I64, "rows must be I32 or I64, got dtype %d", dtype);
  HI3D_REQUIRE(d >= 1 && d <= kMaxRowWidth, "row width must be 1..8, got %d", d);
  HI3D_REQUIRE(n >= 0, "bad n");
  if (n == 0) return HI3D_OK;
  HI3D_REQUIRE(rows && lo && extent && keys, "null pointer argument");
  hipStream_t stream = as_stream(stream_);
  const unsigned blocks = static_cast<unsigned>(ceil_div(n, 256));
  if (dtype == HI3D_I32)
    hipLaunchKernelGGL(pack_rows_kernel<int32_t>, dim3(blocks), dim3(256), 0, stream, static_cast<const int32_t*>(rows),
                       n, d, lo, extent, keys);
  else
    hipLaunchKernelGGL(pack_rows_kernel<int64_t>, dim3(blocks), dim3(256), 0, stream, static_cast<const int64_t*>(rows),
                       n, d, lo, extent, keys);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

extern "C" int hi3d_row_bounds(const void* rows, int32_t dtype, int64_t n, int32_t d, int64_t* lo, int64_t* hi,
                               void* stream_) {
  HI3D_REQUIRE(dtype == HI3D_I32 || dtype == HI3D_I64, "rows must be I32 or I64, got dtype %d", dtype);
  HI3D_REQUIRE(d >= 1 && d <= kMaxRowWidth, "row width must be 1..8, got %d", d);
  HI3D_REQUIRE(n >= 1, "rows must be non-empty");
  HI3D_REQUIRE(rows && lo && hi, "null pointer argument");
  hipStream_t stream = as_stream(stream_);
  hipLaunchKernelGGL(fill_kernel<int64_t>, dim3(1), dim3(64), 0, stream, lo, static_cast<int64_t>(d), INT64_MAX);
  hipLaunchKernelGGL(fill_kernel<int64_t>, dim3(1), dim3(64), 0, stream, hi, static_cast<int64_t>(d), INT64_MIN);
  const int cus = std::max(compute_units(), 1);
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(ceil_div(n, 256), int64_t(cus) * 4));
  if (dtype == HI3D_I32)
    hipLaunchKernelGGL(row_bounds_kernel<int32_t>, dim3(blocks), dim3(256), 0, stream,
                       static_cast<const int32_t*>(rows), n, d, lo, hi);
  else
    hipLaunchKernelGGL(row_bounds_kernel<int64_t>, dim3(blocks), dim3(256), 0, stream,
                       static_cast<const int64_t*>(rows), n, d, lo, hi);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

extern "C" int hi3d_unpack_rows(const int64_t* keys, int64_t n_max, const int64_t* n_dev, int32_t d, const int64_t* lo,
                                const int64_t* extent, void* rows, int32_t dtype, void* stream_) {
  HI3D_REQUIRE(dtype == HI3D_I32 || dtype == HI3D_I64, "rows must be I32 or I64, got dtype %d", dtype);
  HI3D_REQUIRE(d >= 1 && d <= kMaxRowWidth, "row width must be 1..8, got %d", d);
  HI3D_REQUIRE(n_max >= 0, "bad n_max");
  if (n_max == 0) return HI3D_OK;
  HI3D_REQUIRE(keys && n_dev && lo && extent && rows, "null pointer argument");
  hipStream_t stream = as_stream(stream_);
  const unsigned blocks = static_cast<unsigned>(ceil_div(n_max, 256));
  if (dtype == HI3D_I32)
    hipLaunchKernelGGL(unpack_rows_kernel<int32_t>, dim3(blocks), dim3(256), 0, stream, keys, n_dev, d, lo, extent,
                       static_cast<int32_t*>(rows));
  else
    hipLaunchKernelGGL(unpack_rows_kernel<int64_t>, dim3(blocks), dim3(256), 0, stream, keys, n_dev, d, lo, extent,
                       static_cast<int64_t*>(rows));
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}
