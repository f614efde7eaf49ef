// C entry points of the library's radix sort and scan (csrc/radix.h), which the kernel
// map, plan and unique builds use internally.
#include "common.h"
#include "radix.h"

using namespace hi3d;

extern "C" {

int hi3d_sort_pairs_workspace(int64_t n, int64_t* bytes) {
  HI3D_REQUIRE(bytes != nullptr, "bytes_host is NULL");
  HI3D_REQUIRE(n >= 0 && n < (int64_t(1) << 31) - 1, "bad element count");
  *bytes = radix::temp_bytes(n);
  return HI3D_OK;
}

int hi3d_sort_pairs(void* keys, void* keys_alt, int32_t* vals, int32_t* vals_alt, int64_t n, int32_t key_bytes,
                    int32_t begin_bit, int32_t end_bit, void* workspace, int64_t workspace_bytes, int32_t* in_alt,
                    void* stream_) {
  hipStream_t stream = as_stream(stream_);
  HI3D_REQUIRE(key_bytes == 4 || key_bytes == 8, "key_bytes must be 4 or 8, got %d", key_bytes);
  HI3D_REQUIRE(n >= 0 && n < (int64_t(1) << 31) - 1, "bad element count");
  HI3D_REQUIRE(begin_bit >= 0 && begin_bit <= end_bit && end_bit <= 8 * key_bytes, "bad bit range [%d, %d)",
               begin_bit, end_bit);
  HI3D_REQUIRE(in_alt != nullptr, "null pointer argument");
  *in_alt = 0;
  if (n == 0 || begin_bit == end_bit) return HI3D_OK;
  HI3D_REQUIRE(keys && keys_alt && vals && vals_alt && workspace, "null pointer argument");
  HI3D_REQUIRE(workspace_bytes >= radix::temp_bytes(n), "workspace too small: %lld < %lld bytes",
               static_cast<long long>(workspace_bytes), static_cast<long long>(radix::temp_bytes(n)));
  int32_t* v = vals;
  int32_t* va = vals_alt;
  if (key_bytes == 4) {
    auto* k = static_cast<uint32_t*>(keys);
    auto* ka = static_cast<uint32_t*>(keys_alt);
    HI3D_HIP_CHECK(radix::sort_pairs(workspace, workspace_bytes, k, ka, v, va, n, begin_bit, end_bit, stream));
  } else {
    auto* k = static_cast<unsigned long long*>(keys);
    auto* ka = static_cast<unsigned long long*>(keys_alt);
    HI3D_HIP_CHECK(radix::sort_pairs(workspace, workspace_bytes, k, ka, v, va, n, begin_bit, end_bit, stream));
  }
  *in_alt = v == vals ? 0 : 1;
  return HI3D_OK;
}

int hi3d_scan(const int32_t* in, int32_t* out, int64_t n, int32_t inclusive, void* workspace,
              int64_t workspace_bytes, void* stream_) {
  hipStream_t stream = as_stream(stream_);
  HI3D_REQUIRE(n >= 0 && n < (int64_t(1) << 31) - 1, "bad element count");
  if (n == 0) return HI3D_OK;
  HI3D_REQUIRE(in && out && workspace, "null pointer argument");
  HI3D_REQUIRE(workspace_bytes >= radix::temp_bytes(n), "workspace too small: %lld < %lld bytes",
               static_cast<long long>(workspace_bytes), static_cast<long long>(radix::temp_bytes(n)));
  HI3D_HIP_CHECK(radix::scan(workspace, workspace_bytes, in, out, n, inclusive != 0, stream));
  return HI3D_OK;
}

}  // extern "C"
