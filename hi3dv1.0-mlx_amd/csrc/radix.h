// Device-wide sort and scan of the library: an LSD radix sort of (key, int32 value)
// pairs with 8-bit digits, and exclusive / inclusive sums of int32 arrays. Every pass
// runs three kernels over tiles of kTile elements:
//   upsweep    each tile's digit counts, stored digit-major ([digit][tile]);
//   scan       one workgroup per digit turns its row of tile counts into exclusive
//              prefixes and writes the digit's total (skipped for at most kDirect
//              tiles: the downsweep then sums the rows itself);
//   downsweep  each tile ranks its keys stably within the tile (wave-wide ballots
//              match the lanes of equal digit, a running count per wave and digit
//              keeps element order), places them in LDS in digit order and writes
//              each digit's run to digit base + tile prefix, as contiguous stores.
// Passes ping-pong between the caller's two buffers; after an odd number of passes the
// result is in the alternate buffers (the pointers are swapped like a double buffer).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <utility>

#include "common.h"

namespace hi3d {
namespace radix {
namespace {  // each including file gets its own copy of the kernels

constexpr int kThreads = 256;
constexpr int kItems = 16;
constexpr int kTile = kThreads * kItems;
constexpr int kBins = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kDirect = 32;  // tile counts up to which the downsweep sums the rows
static_assert(kBins == kThreads, "one thread per digit in the per-digit steps");

inline int64_t tiles(int64_t n) { return std::max<int64_t>(ceil_div(n, kTile), 1); }

// Workspace bytes of sort_pairs and scan for n elements: per-tile counts and totals.
inline int64_t temp_bytes(int64_t n) { return align_up(tiles(n) * kBins * 4, 256) + align_up(kBins * 4, 256); }

// Exclusive prefix of v over the block's 256 threads; *total gets the sum. part holds
// kWaves ints of LDS; the function ends with a barrier, so part can be reused.
__device__ __forceinline__ int32_t block_exclusive(int32_t v, int32_t* part, int32_t* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int32_t x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int32_t y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63) part[w] = x;
  __syncthreads();
  int32_t off = 0, all = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    const int32_t p = part[i];
    off += i < w ? p : 0;
    all += p;
  }
  *total = all;
  __syncthreads();
  return off + x - v;
}

template <typename K>
__device__ __forceinline__ uint32_t digit_of(K key, int shift, uint32_t dmask) {
  return static_cast<uint32_t>(key >> shift) & dmask;
}

// counts[d * ntiles + t]: keys of tile t with digit d (every digit written).
template <typename K>
__global__ __launch_bounds__(kThreads) void upsweep_kernel(const K* __restrict__ keys, int64_t n, int shift,
                                                           uint32_t dmask, int32_t* __restrict__ counts,
                                                           int64_t ntiles) {
  __shared__ int32_t hist[kWaves][kBins];
  const int t = threadIdx.x, w = t >> 6;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) hist[i][t] = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
  K kv[kItems];
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int64_t e = base + i * kThreads + t;
    kv[i] = e < n ? keys[e] : K(0);
  }
#pragma unroll
  for (int i = 0; i < kItems; ++i)
    if (base + i * kThreads + t < n) atomicAdd(&hist[w][digit_of(kv[i], shift, dmask)], 1);
  __syncthreads();
  int32_t s = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) s += hist[i][t];
  counts[static_cast<int64_t>(t) * ntiles + blockIdx.x] = s;
}

// Row blockIdx.x of counts ([rows][len]) becomes its exclusive prefix; totals[row] its sum.
__global__ __launch_bounds__(kThreads) void row_scan_kernel(int32_t* __restrict__ counts, int64_t len,
                                                            int32_t* __restrict__ totals) {
  __shared__ int32_t part[kWaves];
  int32_t* const row = counts + static_cast<int64_t>(blockIdx.x) * len;
  // thread t owns the contiguous segment [t * per, (t + 1) * per)
  const int64_t per = (len + kThreads - 1) / kThreads;
  const int64_t lo = std::min<int64_t>(threadIdx.x * per, len), hi = std::min<int64_t>(lo + per, len);
  int32_t s = 0;
  for (int64_t i = lo; i < hi; ++i) s += row[i];
  int32_t all;
  int32_t run = block_exclusive(s, part, &all);
  for (int64_t i = lo; i < hi; ++i) {
    const int32_t v = row[i];
    row[i] = run;
    run += v;
  }
  if (threadIdx.x == 0) totals[blockIdx.x] = all;
}

template <typename K>
__global__ __launch_bounds__(kThreads) void downsweep_kernel(const K* __restrict__ keys_in,
                                                             const int32_t* __restrict__ vals_in,
                                                             K* __restrict__ keys_out, int32_t* __restrict__ vals_out,
                                                             int64_t n, int shift, int nbits,
                                                             const int32_t* __restrict__ counts, int64_t ntiles,
                                                             const int32_t* __restrict__ totals) {
  __shared__ K skeys[kTile];
  __shared__ int32_t svals[kTile];
  __shared__ int32_t wcount[kWaves][kBins];  // running, then each wave's offset in the digit
  __shared__ int32_t lstart[kBins];           // the digit's first position in the tile
  __shared__ int32_t gbase[kBins];            // the digit's first output position of the tile
  __shared__ int32_t part[kWaves];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const uint32_t dmask = (1u << nbits) - 1u;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
  const int valid = static_cast<int>(std::min<int64_t>(kTile, n - base));
#pragma unroll
  for (int i = 0; i < kWaves; ++i) wcount[i][t] = 0;
  {
    // totals == nullptr: counts are raw (at most kDirect tiles), so sum the row here
    int32_t tot, pre;
    if (totals != nullptr) {
      tot = totals[t];
      pre = counts[static_cast<int64_t>(t) * ntiles + blockIdx.x];
    } else {
      tot = 0;
      pre = 0;
      for (int b = 0; b < static_cast<int>(ntiles); ++b) {
        const int32_t c = counts[t * ntiles + b];
        tot += c;
        pre += b < static_cast<int>(blockIdx.x) ? c : 0;
      }
    }
    int32_t all;
    const int32_t ex = block_exclusive(tot, part, &all);
    gbase[t] = ex + pre;
  }
  // wave w holds tile elements w * 64 * kItems + 64 i + lane (element order = (w, i, lane));
  // past n a key of all ones, whose digit is the largest, so it ranks after every valid one
  K kv[kItems];
  int32_t vv[kItems], rk[kItems];
  const int64_t wb = base + static_cast<int64_t>(w) * 64 * kItems + lane;
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int64_t e = wb + 64 * i;
    const bool ok = e < n;
    kv[i] = ok ? keys_in[e] : ~K(0);
    vv[i] = ok ? vals_in[e] : 0;
  }
  const uint64_t lt = (uint64_t(1) << lane) - 1u;
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const uint32_t d = digit_of(kv[i], shift, dmask);
    uint64_t peers = ~uint64_t(0);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      if (b < nbits) {
        const bool bit = (d >> b) & 1u;
        const uint64_t bal = __ballot(bit);
        peers &= bit ? bal : ~bal;
      }
    }
    const int32_t before = wcount[w][d];
    const uint64_t below = peers & lt;
    rk[i] = before + __popcll(below);
    if (below == 0) wcount[w][d] = before + __popcll(peers);
  }
  __syncthreads();
  {
    int32_t run = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
      const int32_t c = wcount[i][t];
      wcount[i][t] = run;
      run += c;
    }
    int32_t all;
    lstart[t] = block_exclusive(run, part, &all);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const uint32_t d = digit_of(kv[i], shift, dmask);
    const int p = lstart[d] + wcount[w][d] + rk[i];
    skeys[p] = kv[i];
    svals[p] = vv[i];
  }
  __syncthreads();
  for (int j = t; j < valid; j += kThreads) {
    const K key = skeys[j];
    const uint32_t d = digit_of(key, shift, dmask);
    const int64_t o = gbase[d] + (j - lstart[d]);
    keys_out[o] = key;
    vals_out[o] = svals[j];
  }
}

// Block-wide sort of kThreads * ITEMS (uint32 key, uint32 value) pairs by key bits
// [0, key_bits): thread (wave w, lane) holds elements w * 64 * ITEMS + 64 i + lane in
// keys[i] / vals[i]. On return skeys / svals (LDS, kThreads * ITEMS each) hold the pairs
// in key order (ties in element order). wcount, lstart and part are LDS scratch of
// kWaves x kBins, kBins and kWaves ints.
template <int ITEMS>
__device__ void block_sort_pairs(uint32_t (&keys)[ITEMS], uint32_t (&vals)[ITEMS], int key_bits,
                                 uint32_t* __restrict__ skeys, uint32_t* __restrict__ svals,
                                 int32_t (*__restrict__ wcount)[kBins], int32_t* __restrict__ lstart,
                                 int32_t* __restrict__ part) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const uint64_t lt = (uint64_t(1) << lane) - 1u;
  const int wbase = w * 64 * ITEMS + lane;
  if (key_bits <= 0) {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      skeys[wbase + 64 * i] = keys[i];
      svals[wbase + 64 * i] = vals[i];
    }
    __syncthreads();
    return;
  }
  for (int shift = 0; shift < key_bits; shift += 8) {
    const int nbits = key_bits - shift < 8 ? key_bits - shift : 8;
    const uint32_t dmask = (1u << nbits) - 1u;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) wcount[i][t] = 0;
    __syncthreads();
    int32_t rk[ITEMS];
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const uint32_t d = (keys[i] >> shift) & dmask;
      uint64_t peers = ~uint64_t(0);
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        if (b < nbits) {
          const bool bit = (d >> b) & 1u;
          const uint64_t bal = __ballot(bit);
          peers &= bit ? bal : ~bal;
        }
      }
      const int32_t before = wcount[w][d];
      const uint64_t below = peers & lt;
      rk[i] = before + __popcll(below);
      if (below == 0) wcount[w][d] = before + __popcll(peers);
    }
    __syncthreads();
    {
      int32_t run = 0;
#pragma unroll
      for (int i = 0; i < kWaves; ++i) {
        const int32_t c = wcount[i][t];
        wcount[i][t] = run;
        run += c;
      }
      int32_t all;
      lstart[t] = block_exclusive(run, part, &all);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const uint32_t d = (keys[i] >> shift) & dmask;
      const int p = lstart[d] + wcount[w][d] + rk[i];
      skeys[p] = keys[i];
      svals[p] = vals[i];
    }
    __syncthreads();
    if (shift + 8 < key_bits) {
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) {
        keys[i] = skeys[wbase + 64 * i];
        vals[i] = svals[wbase + 64 * i];
      }
      __syncthreads();
    }
  }
}

// Sorts n (key, value) pairs stably by key bits [begin_bit, end_bit). keys / vals hold
// the input; on return they point at the sorted pairs, which may be the former
// keys_alt / vals_alt (swapped with them). temp: temp_bytes(n) bytes.
template <typename K>
hipError_t sort_pairs(void* temp, int64_t temp_size, K*& keys, K*& keys_alt, int32_t*& vals, int32_t*& vals_alt,
                      int64_t n, int begin_bit, int end_bit, hipStream_t stream) {
  if (n <= 0 || end_bit <= begin_bit) return hipSuccess;
  if (temp_size < temp_bytes(n) || end_bit > static_cast<int>(8 * sizeof(K)) || begin_bit < 0)
    return hipErrorInvalidValue;
  const int64_t nt = tiles(n);
  auto* counts = static_cast<int32_t*>(temp);
  auto* totals = reinterpret_cast<int32_t*>(static_cast<char*>(temp) + align_up(nt * kBins * 4, 256));
  const dim3 grid(static_cast<unsigned>(nt));
  for (int shift = begin_bit; shift < end_bit; shift += 8) {
    const int nbits = std::min(8, end_bit - shift);
    const uint32_t dmask = (1u << nbits) - 1u;
    hipLaunchKernelGGL(upsweep_kernel<K>, grid, dim3(kThreads), 0, stream, keys, n, shift, dmask, counts, nt);
    const bool direct = nt <= kDirect;
    if (!direct)
      hipLaunchKernelGGL(row_scan_kernel, dim3(kBins), dim3(kThreads), 0, stream, counts, nt, totals);
    hipLaunchKernelGGL(downsweep_kernel<K>, grid, dim3(kThreads), 0, stream, keys, vals, keys_alt, vals_alt, n,
                       shift, nbits, counts, nt, direct ? nullptr : totals);
    std::swap(keys, keys_alt);
    std::swap(vals, vals_alt);
  }
  return hipGetLastError();
}

// Per-tile sums of in (tile t's sum at sums[t]).
__global__ __launch_bounds__(kThreads) void tile_sum_kernel(const int32_t* __restrict__ in, int64_t n,
                                                            int32_t* __restrict__ sums) {
  __shared__ int32_t part[kWaves];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
  int32_t s = 0;
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int64_t e = base + i * kThreads + threadIdx.x;
    s += e < n ? in[e] : 0;
  }
  int32_t all;
  block_exclusive(s, part, &all);
  if (threadIdx.x == 0) sums[blockIdx.x] = all;
}

// out = exclusive (or inclusive) prefix sum of in, tile by tile from the tile offsets.
__global__ __launch_bounds__(kThreads) void tile_scan_kernel(const int32_t* __restrict__ in, int64_t n,
                                                             const int32_t* __restrict__ offs, bool inclusive,
                                                             int32_t* __restrict__ out) {
  __shared__ int32_t part[kWaves];
  // thread t owns kItems consecutive elements
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile + static_cast<int64_t>(threadIdx.x) * kItems;
  int32_t v[kItems];
  int32_t s = 0;
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    v[i] = base + i < n ? in[base + i] : 0;
    s += v[i];
  }
  int32_t all;
  int32_t run = offs[blockIdx.x] + block_exclusive(s, part, &all);
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int32_t next = run + v[i];
    if (base + i < n) out[base + i] = inclusive ? next : run;
    run = next;
  }
}

// out[i] = sum of in[0 .. i) (exclusive) or in[0 .. i] (inclusive); out may be in.
// temp: temp_bytes(n) bytes.
inline hipError_t scan(void* temp, int64_t temp_size, const int32_t* in, int32_t* out, int64_t n, bool inclusive,
                       hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  if (temp_size < temp_bytes(n)) return hipErrorInvalidValue;
  const int64_t nt = tiles(n);
  auto* sums = static_cast<int32_t*>(temp);
  auto* total = reinterpret_cast<int32_t*>(static_cast<char*>(temp) + align_up(nt * kBins * 4, 256));
  hipLaunchKernelGGL(tile_sum_kernel, dim3(static_cast<unsigned>(nt)), dim3(kThreads), 0, stream, in, n, sums);
  hipLaunchKernelGGL(row_scan_kernel, dim3(1), dim3(kThreads), 0, stream, sums, nt, total);
  hipLaunchKernelGGL(tile_scan_kernel, dim3(static_cast<unsigned>(nt)), dim3(kThreads), 0, stream, in, n, sums,
                     inclusive, out);
  return hipGetLastError();
}

}  // namespace
}  // namespace radix
}  // namespace hi3d
