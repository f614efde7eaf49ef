// Execution plans of the gather-MFMA convolution.
//
// The convolution is output-stationary: a tile of kTileRows output rows runs one dense
// MFMA contraction per kernel offset that is present in at least one of its rows. To
// keep that union small, output rows are reordered: first by Morton code of their
// coordinates (spatial locality of the gathered rows), then, inside windows of
// `window_rows` Morton-ordered rows, by their 27-bit neighbour-presence mask (radix sort
// is stable, so rows with one mask stay in Morton order). The plan stores per tile the
// output rows, the transposed gather indices [kvol][kTileRows] (one contiguous run per
// offset) and the union mask. Output rows are written once each: the "scatter" is a
// permuted row store, no atomics.
#include <algorithm>

#include "common.h"
#include "conv_tile.h"
#include "radix.h"

namespace hi3d {
namespace {

constexpr int kHaloRows = 256;   // output rows per halo tile
constexpr int kHaloMax = 768;    // halo slots per tile (the last one always absent)
constexpr int kHaloKvol = 27;    // 3x3x3 submanifold maps only

__device__ __forceinline__ uint64_t spread3(uint32_t v) {
  // spread the low 19 bits of v to every third bit
  uint64_t x = v & 0x7ffffu;
  x = (x | (x << 32)) & 0x001f00000000ffffull;
  x = (x | (x << 16)) & 0x001f0000ff0000ffull;
  x = (x | (x << 8)) & 0x100f00f00f00f00full;
  x = (x | (x << 4)) & 0x10c30c30c30c30c3ull;
  x = (x | (x << 2)) & 0x1249249249249249ull;
  return x;
}

// key = batch above the 3 * coord_bits interleaved bits of x, y, z (x highest); K is
// uint32_t when the sorted bits fit 32.
template <typename K>
__global__ void morton_kernel(const int4* __restrict__ coords, int64_t n, int coord_bits, K* __restrict__ keys,
                              int32_t* __restrict__ rows) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int4 c = coords[i];
  uint64_t m = (spread3(static_cast<uint32_t>(c.y)) << 2) | (spread3(static_cast<uint32_t>(c.z)) << 1) |
               spread3(static_cast<uint32_t>(c.w));
  keys[i] = static_cast<K>((static_cast<uint64_t>(static_cast<uint32_t>(c.x) & 0x7f) << (3 * coord_bits)) | m);
  rows[i] = static_cast<int32_t>(i);
}

// Bits of the Morton key to sort on: (coord_bits, batch_bits), 0 = the full 19 and 7.
int morton_sort_bits(int coord_bits, int batch_bits, int* cb) {
  *cb = coord_bits > 0 ? coord_bits : 19;
  return 3 * *cb + (batch_bits > 0 || coord_bits > 0 ? batch_bits : 7);
}

__global__ void iota_kernel(int32_t* __restrict__ rows, int64_t n) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) rows[i] = static_cast<int32_t>(i);
}

// The table rows srow[0 .. nrows) (srow in LDS; -1 = absent row) into LDS as
// [row][kvol], kvol <= 32, nrows <= blockDim.x: consecutive threads read consecutive
// entries of a row, so a wave's loads touch a few rows' contiguous entries instead of
// one entry of 64 scattered rows.
__device__ __forceinline__ void stage_rows(const int32_t* __restrict__ table, const int32_t* __restrict__ srow,
                                           int kvol, int nrows, int32_t absent, int32_t* __restrict__ lds) {
  const int total = nrows * kvol;
  const int bd = blockDim.x;
  auto fetch = [&](int e) -> int32_t {
    const int row = e / kvol;
    const int k = e - row * kvol;
    const int32_t src = srow[row];
    return src >= 0 ? table[static_cast<int64_t>(src) * kvol + k] : absent;
  };
  // all of a thread's (at most 32) loads in flight before their LDS stores
  constexpr int U = 32;
  for (int base = threadIdx.x; base < total; base += U * bd) {
    int32_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = base + u * bd;
      v[u] = e < total ? fetch(e) : 0;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = base + u * bd;
      if (e < total) lds[e] = v[u];
    }
  }
}

// key = (window << 27) | presence-mask key, for rows taken in Morton order.
constexpr int kMaskRows = 256;
// Sort key of a 3x3x3 presence mask: its bits reordered so that the 8 corner offsets
// are the most significant, then the 12 edges, the 6 faces and the centre. On surfaces
// corners are the offsets most often absent, so rows that differ only in edge or face
// neighbours sort next to each other, and a tile that spans two masks runs fewer extra
// offsets (on a 543k-voxel shell set: 1.145 -> 1.105 computed per present pair at
// 2^18-row windows, against sorting the mask itself).
__device__ __forceinline__ uint32_t subm_mask_key(uint32_t mask) {
  // key bit of offset k (k = 9 dx + 3 dy + dz over {0, 1, 2}^3)
  constexpr uint8_t kBit[27] = {26, 18, 25, 17, 6, 16, 24, 15, 23, 14, 5, 13, 4, 0, 3, 12, 2, 11, 22, 10, 21, 9, 1, 8, 20, 7, 19};
  uint32_t key = 0;
#pragma unroll
  for (int k = 0; k < 27; ++k) key |= ((mask >> k) & 1u) << kBit[k];
  return key;
}

// The presence-mask sort key of every row, in row order (the table read as one
// contiguous block per kMaskRows rows). kvol <= 32.
__global__ __launch_bounds__(kMaskRows) void row_mask_kernel(const int32_t* __restrict__ table, int64_t n_out,
                                                             int kvol, int64_t n_in, uint32_t* __restrict__ masks) {
  __shared__ int32_t staged[kMaskRows * 32];
  const int64_t p0 = static_cast<int64_t>(blockIdx.x) * kMaskRows;
  const int rows = static_cast<int>(n_out - p0 < kMaskRows ? n_out - p0 : kMaskRows);
  const int32_t* src = table + p0 * kvol;
  const int total = rows * kvol;
  // fourteen independent loads in flight per thread before their LDS stores
  constexpr int U = 14;
  for (int base = threadIdx.x; base < total; base += U * kMaskRows) {
    int32_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = base + u * kMaskRows;
      v[u] = e < total ? src[e] : 0;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = base + u * kMaskRows;
      if (e < total) staged[e] = v[u];
    }
  }
  __syncthreads();
  if (static_cast<int>(threadIdx.x) >= rows) return;
  const int32_t* t = staged + threadIdx.x * kvol;
  uint32_t mask = 0;
  for (int k = 0; k < kvol; ++k)
    if (static_cast<uint64_t>(static_cast<uint32_t>(t[k])) < static_cast<uint64_t>(n_in)) mask |= 1u << k;
  masks[p0 + threadIdx.x] = kvol == 27 ? subm_mask_key(mask) : mask;
}

// masks: the rows' mask keys in row order (NULL: no mask, kvol > 32).
template <typename K>
__global__ void mask_keys_kernel(const uint32_t* __restrict__ masks, int64_t n_out, int mask_bits,
                                 const int32_t* __restrict__ order, int64_t window, K* __restrict__ keys,
                                 int32_t* __restrict__ rows) {
  const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (p >= n_out) return;
  const int32_t row = order[p];
  const uint64_t w = window > 0 ? static_cast<uint64_t>(p / window) : 0;
  keys[p] = static_cast<K>((w << mask_bits) | (masks != nullptr ? masks[row] : 0u));
  rows[p] = row;
}

// One block of kTileRows threads per tile: output rows, transposed gather indices and
// the union mask.
__global__ __launch_bounds__(kTileRows) void tile_kernel(const int32_t* __restrict__ table, int64_t n_out,
                                                         int kvol, int64_t n_in,
                                                         const int32_t* __restrict__ order,
                                                         int32_t* __restrict__ rows,
                                                         int32_t* __restrict__ gidx,
                                                         uint32_t* __restrict__ tile_mask) {
  __shared__ uint32_t wave_mask[kTileRows / 64];
  __shared__ int32_t staged[kTileRows * 32];
  __shared__ int32_t srow[kTileRows];
  const int64_t tile = blockIdx.x;
  const int r = threadIdx.x;
  const int64_t p = tile * kTileRows + r;
  const int32_t row = p < n_out ? order[p] : -1;
  rows[p] = row;
  uint32_t mask = 0;
  int32_t* g = gidx + tile * kvol * kTileRows + r;
  const int32_t absent = static_cast<int32_t>(n_in);
  if (kvol <= 32) {
    srow[r] = row;
    __syncthreads();
    stage_rows(table, srow, kvol, kTileRows, absent, staged);
    __syncthreads();
    const int32_t* t = staged + r * kvol;
    for (int k = 0; k < kvol; ++k) {
      int32_t v = t[k];
      if (static_cast<uint64_t>(static_cast<uint32_t>(v)) >= static_cast<uint64_t>(n_in)) v = absent;
      g[k * kTileRows] = v;
      if (v != absent) mask |= 1u << k;
    }
  } else {
    for (int k = 0; k < kvol; ++k) {
      int32_t v = absent;
      if (row >= 0) {
        v = table[static_cast<int64_t>(row) * kvol + k];
        if (static_cast<uint64_t>(static_cast<uint32_t>(v)) >= static_cast<uint64_t>(n_in)) v = absent;
      }
      g[k * kTileRows] = v;
    }
  }
  // OR-reduce over the wave, then over the block
  for (int d = 32; d >= 1; d >>= 1) mask |= __shfl_xor(mask, d, 64);
  if ((r & 63) == 0) wave_mask[r >> 6] = mask;
  __syncthreads();
  if (r == 0) {
    uint32_t m = 0;
    for (int w = 0; w < kTileRows / 64; ++w) m |= wave_mask[w];
    tile_mask[tile] = kvol <= 32 ? m : 0xffffffffu;
  }
}

// Halo plans (27-offset submanifold maps): tiles of kHaloRows output rows in Morton
// order. Per tile: its output rows, the sorted unique input rows its offsets touch (the
// halo, padded with the absent id n_in; at most kHaloMax - 1 used so that the last slot
// always reads as a zero row), each (row, offset)'s position in the halo (0xffff when
// absent) laid out [row][32] (offsets 0..26), and per 32-row block the 27-bit mask of
// offsets present in any of its rows. A tile whose halo does not fit sets *overflow.
__global__ __launch_bounds__(kHaloRows) void halo_tile_kernel(const int32_t* __restrict__ table, int64_t n_out,
                                                              int64_t n_in, const int32_t* __restrict__ order,
                                                              int key_bits, int32_t* __restrict__ rows,
                                                              int32_t* __restrict__ halo, int32_t* __restrict__ hcount,
                                                              uint16_t* __restrict__ loff, uint32_t* __restrict__ bmask,
                                                              int32_t* __restrict__ overflow) {
  static_assert(kHaloRows == radix::kThreads, "the block sort runs one thread per tile row");
  __shared__ uint32_t sorted[kHaloRows * kHaloKvol];
  __shared__ uint32_t sorted_vals[kHaloRows * kHaloKvol];
  __shared__ int32_t wcount[radix::kWaves][radix::kBins];
  __shared__ int32_t lstart[radix::kBins];
  __shared__ int32_t part[radix::kWaves];
  const int64_t tile = blockIdx.x;
  const int r = threadIdx.x;
  const int64_t p = tile * kHaloRows + r;
  const int32_t row = p < n_out ? order[p] : -1;
  rows[p] = row;
  const uint32_t absent = static_cast<uint32_t>(n_in);
  uint32_t keys[kHaloKvol], vals[kHaloKvol];
  uint32_t mask = 0;
#pragma unroll
  for (int k = 0; k < kHaloKvol; ++k) {
    uint32_t v = absent;
    if (row >= 0) {
      const uint32_t t = static_cast<uint32_t>(table[static_cast<int64_t>(row) * kHaloKvol + k]);
      if (t < absent) {
        v = t;
        mask |= 1u << k;
      }
    }
    keys[k] = v;
    vals[k] = static_cast<uint32_t>(r * 32 + k);  // position in the [row][32] layout
  }
  // 32-row block masks
#pragma unroll
  for (int d = 16; d >= 1; d >>= 1) mask |= __shfl_xor(mask, d, 64);
  if ((r & 31) == 0) bmask[tile * (kHaloRows / 32) + (r >> 5)] = mask;
  radix::block_sort_pairs(keys, vals, key_bits, sorted, sorted_vals, wcount, lstart, part);
  // thread r takes sorted ranks r*27 .. r*27+26
#pragma unroll
  for (int i = 0; i < kHaloKvol; ++i) {
    keys[i] = sorted[r * kHaloKvol + i];
    vals[i] = sorted_vals[r * kHaloKvol + i];
  }
  int heads = 0;
#pragma unroll
  for (int i = 0; i < kHaloKvol; ++i) {
    const int pos = r * kHaloKvol + i;
    const uint32_t prev = pos > 0 ? sorted[pos - 1] : 0xffffffffu;
    heads += (keys[i] < absent && keys[i] != prev) ? 1 : 0;
  }
  int total = 0;
  const int base = radix::block_exclusive(heads, part, &total);
  uint16_t* lt = loff + tile * kHaloRows * 32;
  int32_t* ht = halo + tile * kHaloMax;
  int run = base - 1;  // halo position of the current run
#pragma unroll
  for (int i = 0; i < kHaloKvol; ++i) {
    const int pos = r * kHaloKvol + i;
    const uint32_t prev = pos > 0 ? sorted[pos - 1] : 0xffffffffu;
    const bool present = keys[i] < absent;
    if (present && keys[i] != prev) {
      ++run;
      if (run < kHaloMax - 1) ht[run] = static_cast<int32_t>(keys[i]);
    }
    lt[vals[i]] = (present && run < kHaloMax - 1) ? static_cast<uint16_t>(run) : static_cast<uint16_t>(0xffff);
  }
  // unused positions of the [row][32] layout and of the halo
  for (int k = kHaloKvol; k < 32; ++k) lt[r * 32 + k] = 0xffff;
  for (int i = total + r; i < kHaloMax; i += kHaloRows) ht[i] = static_cast<int32_t>(absent);
  if (r == 0) {
    hcount[tile] = total < kHaloMax - 1 ? total : kHaloMax - 1;
    if (total > kHaloMax - 1) atomicOr(overflow, 1);
  }
}

int64_t sort_temp_bytes(int64_t n) { return radix::temp_bytes(std::max<int64_t>(n, 1)); }

// Sorts (keys, rows) on key bits [0, bits) with 32-bit keys when they fit, else 64-bit
// ones; kbuf0 / kbuf1 hold n 64-bit keys each, rows start in r0. fill(k) launches the
// kernel that writes the keys into k (uint32_t* or unsigned long long*) and the rows
// into r0. *sorted receives the sorted rows (r0 or r1).
template <typename Fill>
hipError_t sort_rows(void* temp, int64_t temp_bytes, unsigned long long* kbuf0, unsigned long long* kbuf1, int32_t* r0,
                     int32_t* r1, int n, int bits, hipStream_t stream, Fill fill, const int32_t** sorted) {
  hipError_t e;
  if (bits <= 32) {
    auto* k0 = reinterpret_cast<uint32_t*>(kbuf0);
    auto* k1 = reinterpret_cast<uint32_t*>(kbuf1);
    fill(k0);
    e = radix::sort_pairs(temp, temp_bytes, k0, k1, r0, r1, n, 0, std::max(bits, 1), stream);
  } else {
    fill(kbuf0);
    e = radix::sort_pairs(temp, temp_bytes, kbuf0, kbuf1, r0, r1, n, 0, bits, stream);
  }
  *sorted = r0;
  return e;
}

}  // namespace
}  // namespace hi3d

using namespace hi3d;

extern "C" {

int32_t hi3d_conv_tile_rows(void) { return kTileRows; }

int hi3d_conv_plan_workspace(int64_t n_out, int64_t* bytes) {
  HI3D_REQUIRE(bytes != nullptr, "bytes_host is NULL");
  HI3D_REQUIRE(n_out >= 0 && n_out < (int64_t(1) << 31) - 1, "bad n_out");
  const int64_t m = std::max<int64_t>(n_out, 1);
  *bytes = 2 * align_up(m * 8, 256) + 3 * align_up(m * 4, 256) + sort_temp_bytes(m) + 256;
  return HI3D_OK;
}

int hi3d_conv_plan(const int32_t* table, int64_t n_out, int32_t kvol, int64_t n_in, const int32_t* coords,
                   int32_t coord_bits, int32_t batch_bits, int64_t window_rows, void* workspace,
                   int64_t workspace_bytes, int32_t* rows, int32_t* gidx, uint32_t* tile_mask, void* stream_) {
  hipStream_t stream = as_stream(stream_);
  int64_t need = 0;
  int rc = hi3d_conv_plan_workspace(n_out, &need);
  if (rc != HI3D_OK) return rc;
  HI3D_REQUIRE(kvol >= 1 && kvol <= 1024, "kvol out of range: %d", kvol);
  HI3D_REQUIRE(n_in >= 0 && n_in < (int64_t(1) << 31) - 1, "bad n_in");
  HI3D_REQUIRE(coord_bits >= 0 && coord_bits <= 19 && batch_bits >= 0 && batch_bits <= 7,
               "coord_bits must be in [0, 19] and batch_bits in [0, 7]");
  if (n_out == 0) return HI3D_OK;
  HI3D_REQUIRE(table && rows && gidx && tile_mask && workspace, "null pointer argument");
  HI3D_REQUIRE(workspace_bytes >= need, "workspace too small");
  Workspace ws(workspace, workspace_bytes);
  auto* k0 = ws.take<unsigned long long>(n_out);
  auto* k1 = ws.take<unsigned long long>(n_out);
  auto* r0 = ws.take<int32_t>(n_out);
  auto* r1 = ws.take<int32_t>(n_out);
  auto* masks = ws.take<uint32_t>(n_out);
  const int64_t temp_bytes = sort_temp_bytes(n_out);
  void* temp = ws.take<char>(temp_bytes);
  const unsigned blocks = static_cast<unsigned>(ceil_div(n_out, 256));
  const int n = static_cast<int>(n_out);
  const int32_t* order = nullptr;
  if (coords) {
    int cb = 0;
    const int morton_bits = morton_sort_bits(coord_bits, batch_bits, &cb);
    const int4* c4 = reinterpret_cast<const int4*>(coords);
    HI3D_HIP_CHECK(sort_rows(
        temp, temp_bytes, k0, k1, r0, r1, n, morton_bits, stream,
        [&](auto* k) { hipLaunchKernelGGL(morton_kernel, dim3(blocks), dim3(256), 0, stream, c4, n_out, cb, k, r0); },
        &order));
  } else {
    hipLaunchKernelGGL(iota_kernel, dim3(blocks), dim3(256), 0, stream, r0, n_out);
    order = r0;
  }
  // second key: (window, mask); the sort is stable, so Morton order survives inside
  int32_t* ord_in = const_cast<int32_t*>(order);
  int32_t* ord_alt = (ord_in == r0) ? r1 : r0;
  const int mask_bits = kvol <= 32 ? kvol : 0;
  if (mask_bits > 0)
    hipLaunchKernelGGL(row_mask_kernel, dim3(static_cast<unsigned>(ceil_div(n_out, kMaskRows))), dim3(kMaskRows), 0,
                       stream, table, n_out, kvol, n_in, masks);
  const int64_t windows = window_rows > 0 ? ceil_div(n_out, window_rows) : 1;
  int window_bits = 0;
  while ((int64_t(1) << window_bits) < windows) ++window_bits;
  const uint32_t* mk = mask_bits > 0 ? masks : nullptr;
  const int32_t* final_order = nullptr;
  auto fill = [&](auto* k) {
    hipLaunchKernelGGL(mask_keys_kernel, dim3(blocks), dim3(256), 0, stream, mk, n_out, mask_bits, ord_in,
                       window_rows, k, ord_alt);
  };
  if (mask_bits + window_bits > 0) {
    // mask in bits [0, mask_bits), window above it
    HI3D_HIP_CHECK(sort_rows(temp, temp_bytes, k0, k1, ord_alt, ord_in, n, mask_bits + window_bits, stream, fill,
                             &final_order));
  } else {
    fill(reinterpret_cast<uint32_t*>(k0));
    final_order = ord_alt;
  }
  const int64_t ntiles = ceil_div(n_out, kTileRows);
  hipLaunchKernelGGL(tile_kernel, dim3(static_cast<unsigned>(ntiles)), dim3(kTileRows), 0, stream, table, n_out,
                     kvol, n_in, final_order, rows, gidx, tile_mask);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}


int hi3d_halo_plan_workspace(int64_t n_out, int64_t* bytes) {
  return hi3d_conv_plan_workspace(n_out, bytes);
}

int hi3d_halo_plan(const int32_t* table, int64_t n_out, int32_t kvol, int64_t n_in, const int32_t* coords,
                   int32_t coord_bits, int32_t batch_bits, void* workspace, int64_t workspace_bytes, int32_t* rows,
                   int32_t* halo, int32_t* hcount, uint16_t* loff, uint32_t* bmask, int32_t* overflow,
                   void* stream_) {
  hipStream_t stream = as_stream(stream_);
  int64_t need = 0;
  int rc = hi3d_halo_plan_workspace(n_out, &need);
  if (rc != HI3D_OK) return rc;
  HI3D_REQUIRE(kvol == kHaloKvol, "halo plans cover 27-offset maps (got %d offsets)", kvol);
  HI3D_REQUIRE(n_in >= 0 && n_in < (int64_t(1) << 31) - 1, "bad n_in");
  HI3D_REQUIRE(coord_bits >= 0 && coord_bits <= 19 && batch_bits >= 0 && batch_bits <= 7,
               "coord_bits must be in [0, 19] and batch_bits in [0, 7]");
  HI3D_REQUIRE(overflow != nullptr, "null pointer argument");
  launch_fill(overflow, 1, int32_t(0), stream);
  if (n_out == 0) return HI3D_OK;
  HI3D_REQUIRE(table && rows && halo && hcount && loff && bmask && workspace, "null pointer argument");
  HI3D_REQUIRE(workspace_bytes >= need, "workspace too small");
  Workspace ws(workspace, workspace_bytes);
  auto* k0 = ws.take<unsigned long long>(n_out);
  auto* k1 = ws.take<unsigned long long>(n_out);
  auto* r0 = ws.take<int32_t>(n_out);
  auto* r1 = ws.take<int32_t>(n_out);
  const int64_t temp_bytes = sort_temp_bytes(n_out);
  void* temp = ws.take<char>(temp_bytes);
  const unsigned blocks = static_cast<unsigned>(ceil_div(n_out, 256));
  const int32_t* order = r0;
  if (coords) {
    int cb = 0;
    const int morton_bits = morton_sort_bits(coord_bits, batch_bits, &cb);
    const int4* c4 = reinterpret_cast<const int4*>(coords);
    HI3D_HIP_CHECK(sort_rows(
        temp, temp_bytes, k0, k1, r0, r1, static_cast<int>(n_out), morton_bits, stream,
        [&](auto* k) { hipLaunchKernelGGL(morton_kernel, dim3(blocks), dim3(256), 0, stream, c4, n_out, cb, k, r0); },
        &order));
  } else {
    hipLaunchKernelGGL(iota_kernel, dim3(blocks), dim3(256), 0, stream, r0, n_out);
  }
  int key_bits = 1;
  while (key_bits < 32 && (int64_t(1) << key_bits) <= n_in) ++key_bits;
  const int64_t ntiles = ceil_div(n_out, kHaloRows);
  hipLaunchKernelGGL(halo_tile_kernel, dim3(static_cast<unsigned>(ntiles)), dim3(kHaloRows), 0, stream, table, n_out,
                     n_in, order, key_bits, rows, halo, hcount, loff, bmask, overflow);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

int32_t hi3d_halo_tile_rows(void) { return kHaloRows; }
int32_t hi3d_halo_capacity(void) { return kHaloMax; }

}  // extern "C"
