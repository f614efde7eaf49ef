// Kernel maps of the sparse convolutions on gfx950.
//
//  * hash build + probe -> dense [N, K] neighbour table and per-offset counts
//    (reference: _voxel_keys / subm_pairs, src/hi3d_mac/torch_backend/sparse_conv.py:109-149;
//    neighbour_table, src/hi3d_mac/mlx_backend/sparse.py:29-43);
//  * per-offset pair lists by a stable ballot/prefix compaction
//    (reference: _PairTable / get_indice_pairs, sparse_conv.py:37-50,264-283);
//  * the 2x2x2/s2 coarse structure by radix sort + run heads
//    (reference: downsample_structure, src/hi3d_mac/mlx_backend/sparse.py:217-233);
//  * the octree child table from the parent table (reference: child_neighbour_table,
//    src/hi3d_mac/mlx_backend/sparse.py:46-95).
//
// The hash is open addressing with linear probing in HBM. A 32-bit key (key space below
// 2^32 - 1) and its row share one 64-bit slot, so one 64-bit CAS inserts both; wider keys
// use a 64-bit key array plus a row array. Probing writes each (row, offset) cell of the
// table exactly once, so the table does not depend on insertion order.
//
// Slots keep locality: a voxel's home slot is 8 * mix64(its 2x2x2 brick) + its corner in
// the brick, so the eight cells of a brick share one 64-byte run of slots and a row's 26
// neighbours fall in at most 8 such runs.
//
// The map build's own hash is the brick hash below (one bucket per occupied brick, homes
// grouped per 8x8x8-cell superblock); with a workspace for it, its rows are first sorted
// by their superblock-major cell keys and the insert and the probe walk them in that
// order (probe chunks taken XCD by XCD), so neighbouring rows touch the same buckets while
// they sit in L2.

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <mutex>

#include "common.h"
#include "radix.h"

namespace hi3d {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

namespace {

constexpr uint64_t kEmpty = ~0ull;
constexpr int kMaxKvol = 343;  // ksize <= 7

// MurmurHash3's 64-bit finaliser: a bijective mix of the packed key.
__device__ __forceinline__ uint64_t mix64(uint64_t x) {
  x ^= x >> 33;
  x *= 0xff51afd7ed558ccdull;
  x ^= x >> 33;
  x *= 0xc4ceb9fe1a85ec53ull;
  x ^= x >> 33;
  return x;
}

struct Grid {
  int32_t sx, sy, sz, batch;
  __device__ __forceinline__ bool inside(int b, int x, int y, int z) const {
    return static_cast<unsigned>(b) < static_cast<unsigned>(batch) &&
           static_cast<unsigned>(x) < static_cast<unsigned>(sx) &&
           static_cast<unsigned>(y) < static_cast<unsigned>(sy) &&
           static_cast<unsigned>(z) < static_cast<unsigned>(sz);
  }
  __device__ __forceinline__ uint64_t key(int b, int x, int y, int z) const {
    return ((static_cast<uint64_t>(b) * sx + x) * sy + y) * sz + z;
  }
  // the cell's 2x2x2 brick (packed like the cell key over the halved extents) and its
  // corner in the brick
  __device__ __forceinline__ uint64_t brick(int b, int x, int y, int z) const {
    const uint64_t hx = (static_cast<uint64_t>(sx) + 1) >> 1, hy = (static_cast<uint64_t>(sy) + 1) >> 1,
                   hz = (static_cast<uint64_t>(sz) + 1) >> 1;
    return ((static_cast<uint64_t>(b) * hx + (x >> 1)) * hy + (y >> 1)) * hz + (z >> 1);
  }
  __device__ __forceinline__ int corner(int x, int y, int z) const {
    return ((x & 1) << 2) | ((y & 1) << 1) | (z & 1);
  }
  // brick key from brick coordinates (in range)
  __device__ __forceinline__ uint64_t brick_key(int b, int64_t bx, int64_t by, int64_t bz) const {
    const uint64_t hx = (static_cast<uint64_t>(sx) + 1) >> 1, hy = (static_cast<uint64_t>(sy) + 1) >> 1,
                   hz = (static_cast<uint64_t>(sz) + 1) >> 1;
    return ((static_cast<uint64_t>(b) * hx + bx) * hy + by) * hz + bz;
  }
  // the 4x4x4-brick superblock (8x8x8 cells) holding a brick, packed over the quartered
  // brick extents
  __device__ __forceinline__ uint64_t superblock(int b, int64_t bx, int64_t by, int64_t bz) const {
    const uint64_t qx = ((static_cast<uint64_t>(sx) + 1) / 2 + 3) >> 2,
                   qy = ((static_cast<uint64_t>(sy) + 1) / 2 + 3) >> 2,
                   qz = ((static_cast<uint64_t>(sz) + 1) / 2 + 3) >> 2;
    return ((static_cast<uint64_t>(b) * qx + (bx >> 2)) * qy + (by >> 2)) * qz + (bz >> 2);
  }
  // superblock-major cell key: superblock, then the brick's place in it (6 bits), then
  // the cell's corner in the brick (3 bits)
  __device__ __forceinline__ uint64_t sb_cell_key(int b, int x, int y, int z) const {
    const int bx = x >> 1, by = y >> 1, bz = z >> 1;
    return (superblock(b, bx, by, bz) << 9) |
           static_cast<uint64_t>((((bx & 3) << 4) | ((by & 3) << 2) | (bz & 3)) << 3) |
           static_cast<uint64_t>(corner(x, y, z));
  }
  // (batch, x, y, z) of a superblock-major cell key below 2^32
  __device__ __forceinline__ int4 sb_cell_decode(uint32_t key) const {
    const uint32_t qx = static_cast<uint32_t>((((static_cast<uint64_t>(sx) + 1) / 2) + 3) >> 2),
                   qy = static_cast<uint32_t>((((static_cast<uint64_t>(sy) + 1) / 2) + 3) >> 2),
                   qz = static_cast<uint32_t>((((static_cast<uint64_t>(sz) + 1) / 2) + 3) >> 2);
    uint32_t sb = key >> 9;
    const uint32_t pz = sb % qz;
    sb /= qz;
    const uint32_t py = sb % qy;
    sb /= qy;
    const uint32_t px = sb % qx;
    const uint32_t b = sb / qx;
    const uint32_t local = (key >> 3) & 63u, cn = key & 7u;
    const uint32_t bx = (px << 2) | (local >> 4), by = (py << 2) | ((local >> 2) & 3u), bz = (pz << 2) | (local & 3u);
    return make_int4(static_cast<int>(b), static_cast<int>((bx << 1) | (cn >> 2)),
                     static_cast<int>((by << 1) | ((cn >> 1) & 1u)), static_cast<int>((bz << 1) | (cn & 1u)));
  }
  // home bucket of a brick: the superblock's run of 64 buckets (at a hashed, aligned
  // start) at the brick's place in the superblock, so the words and rows of neighbouring
  // bricks share cache lines
  __device__ __forceinline__ uint64_t brick_home(int b, int64_t bx, int64_t by, int64_t bz, uint64_t mask) const {
    const uint64_t local = static_cast<uint64_t>(((bx & 3) << 4) | ((by & 3) << 2) | (bz & 3));
    return ((mix64(superblock(b, bx, by, bz)) << 6) | local) & mask;
  }
  // voxel-slot home: the cell's corner within a run of 8 slots per brick
  __device__ __forceinline__ uint64_t home(int b, int x, int y, int z, uint64_t mask) const {
    return ((mix64(brick(b, x, y, z)) << 3) | static_cast<uint64_t>(corner(x, y, z))) & mask;
  }
};

// perm (optional): visit rows perm[0 ..] (cell order; a negative entry stands for an
// out-of-range row, already flagged) instead of 0 ..
__global__ void insert32_kernel(const int4* __restrict__ coords, int64_t n, Grid g, const int32_t* __restrict__ perm,
                                unsigned long long* __restrict__ slots, uint64_t mask,
                                int32_t* __restrict__ status) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  if (perm != nullptr) {
    const int32_t p = perm[i];
    if (p < 0) return;
    i = p;
  }
  int4 c = coords[i];
  if (!g.inside(c.x, c.y, c.z, c.w)) {
    atomicOr(status, HI3D_MAP_RANGE);
    return;
  }
  uint32_t key = static_cast<uint32_t>(g.key(c.x, c.y, c.z, c.w));
  unsigned long long packed = (static_cast<unsigned long long>(key) << 32) | static_cast<uint32_t>(i);
  uint64_t h = g.home(c.x, c.y, c.z, c.w, mask);
  for (uint64_t probe = 0; probe <= mask; ++probe) {
    unsigned long long prev = atomicCAS(&slots[h], kEmpty, packed);
    if (prev == kEmpty) return;
    if (static_cast<uint32_t>(prev >> 32) == key) {
      atomicOr(status, HI3D_MAP_DUPLICATE);
      return;
    }
    h = (h + 1) & mask;
  }
  atomicOr(status, HI3D_MAP_OVERFLOW);
}

__global__ void insert64_kernel(const int4* __restrict__ coords, int64_t n, Grid g, const int32_t* __restrict__ perm,
                                unsigned long long* __restrict__ keys, int32_t* __restrict__ vals,
                                uint64_t mask, int32_t* __restrict__ status) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  if (perm != nullptr) {
    const int32_t p = perm[i];
    if (p < 0) return;
    i = p;
  }
  int4 c = coords[i];
  if (!g.inside(c.x, c.y, c.z, c.w)) {
    atomicOr(status, HI3D_MAP_RANGE);
    return;
  }
  unsigned long long key = g.key(c.x, c.y, c.z, c.w);
  uint64_t h = g.home(c.x, c.y, c.z, c.w, mask);
  for (uint64_t probe = 0; probe <= mask; ++probe) {
    unsigned long long prev = atomicCAS(&keys[h], kEmpty, key);
    if (prev == kEmpty) {
      vals[h] = static_cast<int32_t>(i);
      return;
    }
    if (prev == key) {
      atomicOr(status, HI3D_MAP_DUPLICATE);
      return;
    }
    h = (h + 1) & mask;
  }
  atomicOr(status, HI3D_MAP_OVERFLOW);
}

__device__ __forceinline__ int32_t lookup32(const unsigned long long* __restrict__ slots,
                                            uint64_t mask, uint64_t h, uint32_t key, int32_t absent) {
  for (uint64_t probe = 0; probe <= mask; ++probe) {
    unsigned long long s = slots[h];
    if (s == kEmpty) return absent;
    if (static_cast<uint32_t>(s >> 32) == key) return static_cast<int32_t>(static_cast<uint32_t>(s));
    h = (h + 1) & mask;
  }
  return absent;
}

__device__ __forceinline__ int32_t lookup64(const unsigned long long* __restrict__ keys,
                                            const int32_t* __restrict__ vals, uint64_t mask, uint64_t h,
                                            unsigned long long key, int32_t absent) {
  for (uint64_t probe = 0; probe <= mask; ++probe) {
    unsigned long long s = keys[h];
    if (s == kEmpty) return absent;
    if (s == key) return vals[h];
    h = (h + 1) & mask;
  }
  return absent;
}

// One block handles kProbeRows rows x kvol offsets; flat (row, offset) order makes the
// table writes coalesced. The block's rows and coordinates are staged in LDS once; each
// thread then takes its cells kProbeBatch at a time, issuing the home-slot loads of all
// of them before resolving any (independent loads in flight instead of one dependent
// chain per cell); a key found past its home slot continues the linear probe there.
// Counts are reduced in LDS, then one atomic per offset per block.
constexpr int kProbeRows = 64;
constexpr int kProbeBatch = 8;

// perm (optional): the block's rows are perm[row0 ..] (cell order; a negative entry p
// stands for the out-of-range row ~p), with the row chunks taken XCD by XCD (block b
// runs on XCD b % 8 and takes chunk (b % 8) * per + b / 8), so each XCD's L2 sees a
// contiguous run of cells.
template <bool kKey64>
__global__ __launch_bounds__(256) void probe_kernel(const int4* __restrict__ coords, int64_t n,
                                                    Grid g, int ksize, const int32_t* __restrict__ perm, int per,
                                                    const unsigned long long* __restrict__ slots,
                                                    const int32_t* __restrict__ vals, uint64_t mask,
                                                    int32_t* __restrict__ nbr,
                                                    int32_t* __restrict__ counts) {
  __shared__ int32_t cnt[kMaxKvol];
  __shared__ int4 sc[kProbeRows];
  __shared__ int32_t so[kProbeRows];
  const int kvol = ksize * ksize * ksize;
  const int half = ksize / 2;
  const int center = kvol / 2;
  const int64_t chunk = perm != nullptr ? static_cast<int64_t>(blockIdx.x % 8) * per + blockIdx.x / 8 : blockIdx.x;
  const int64_t row0 = chunk * kProbeRows;
  if (row0 >= n) return;  // the XCD order's spare blocks (before any barrier)
  const int rows = static_cast<int>(n - row0 < kProbeRows ? n - row0 : kProbeRows);
  for (int k = threadIdx.x; k < kvol; k += blockDim.x) cnt[k] = 0;
  if (threadIdx.x < rows) {
    int64_t o = row0 + threadIdx.x;
    if (perm != nullptr) {
      const int32_t p = perm[o];
      o = p >= 0 ? p : ~p;
    }
    so[threadIdx.x] = static_cast<int32_t>(o);
    sc[threadIdx.x] = coords[o];
  }
  __syncthreads();
  const int cells = rows * kvol;
  const int32_t absent = static_cast<int32_t>(n);
  for (int base = threadIdx.x; base < cells; base += blockDim.x * kProbeBatch) {
    uint64_t h[kProbeBatch], key[kProbeBatch];
    unsigned long long v[kProbeBatch];
    bool look[kProbeBatch];
#pragma unroll
    for (int u = 0; u < kProbeBatch; ++u) {
      const int j = base + u * blockDim.x;
      look[u] = false;
      h[u] = 0;
      key[u] = 0;
      if (j < cells) {
        const int r = j / kvol;
        const int k = j - r * kvol;
        const int4 c = sc[r];
        const int x = c.y + k / (ksize * ksize) - half;
        const int y = c.z + (k / ksize) % ksize - half;
        const int z = c.w + k % ksize - half;
        if (k != center && g.inside(c.x, x, y, z)) {
          look[u] = true;
          h[u] = g.home(c.x, x, y, z, mask);
          key[u] = g.key(c.x, x, y, z);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kProbeBatch; ++u) v[u] = look[u] ? slots[h[u]] : kEmpty;
#pragma unroll
    for (int u = 0; u < kProbeBatch; ++u) {
      const int j = base + u * blockDim.x;
      if (j >= cells) continue;
      const int r = j / kvol;
      const int k = j - r * kvol;
      const int32_t o = so[r];
      int32_t found = absent;
      if (k == center) {
        found = o;
      } else if (look[u]) {
        // the home slot's value is in v; an empty slot ends the probe, a match ends it
        // with the row, another key moves on to the next slots
        if (kKey64) {
          if (v[u] == key[u]) found = vals[h[u]];
          else if (v[u] != kEmpty)
            found = lookup64(slots, vals, mask, (h[u] + 1) & mask, key[u], absent);
        } else {
          const uint32_t k32 = static_cast<uint32_t>(key[u]);
          if (static_cast<uint32_t>(v[u] >> 32) == k32 && v[u] != kEmpty)
            found = static_cast<int32_t>(static_cast<uint32_t>(v[u]));
          else if (v[u] != kEmpty)
            found = lookup32(slots, mask, (h[u] + 1) & mask, k32, absent);
        }
      }
      nbr[static_cast<int64_t>(o) * kvol + k] = found;
      if (found != absent) atomicAdd(&cnt[k], 1);
    }
  }
  __syncthreads();
  for (int k = threadIdx.x; k < kvol; k += blockDim.x)
    if (cnt[k]) atomicAdd(&counts[k], cnt[k]);
}

// ------------------------------------------------------------- brick hash --
// The map build's hash (hi3d_kmap_subm): one bucket per occupied 2x2x2 brick, open
// addressing over buckets (homes grouped per 8x8x8-cell superblock, collisions by double
// hashing; see brick_home and brick_step). A bucket is one 64-bit word, the brick
// key shifted left by 8 with the occupancy mask of its 8 cells in the low byte, plus the
// rows of its 8 cells (rows[8 h ..], valid where the mask bit is set, so only the words
// are cleared per build). A row's 26 neighbours lie in 8 bricks; a lookup reads one word
// (longer probes are rare at the default capacity of one bucket per voxel) and, for a
// present neighbour only, its row. Brick keys must stay below 2^56 - 1.
constexpr unsigned long long kEmptyBrick = ~0ull;

struct BrickTable {
  unsigned long long* words;  // key << 8 | mask, kEmptyBrick when free
  int32_t* rows;
  uint64_t mask;
};

// Collisions probe by double hashing: from the home on in steps of an odd stride drawn
// from the brick key (so the probe sequence visits every bucket of the power-of-two
// table). Linear probing from the clustered superblock runs made long chains.
__device__ __forceinline__ uint64_t brick_step(unsigned long long bk, uint64_t mask) {
  return (mix64(bk ^ 0x9E3779B97F4A7C15ull) | 1ull) & mask;
}

__device__ __forceinline__ unsigned long long shfl_u64(unsigned long long v, int src) {
  const uint32_t lo = static_cast<uint32_t>(__shfl(static_cast<int>(static_cast<uint32_t>(v)), src, 64));
  const uint32_t hi = static_cast<uint32_t>(__shfl(static_cast<int>(static_cast<uint32_t>(v >> 32)), src, 64));
  return (static_cast<unsigned long long>(hi) << 32) | lo;
}

// perm (optional): rows perm[0 ..] in superblock order (a negative entry stands for an
// out-of-range row, already flagged). The lanes of a wave are grouped by brick first (a
// wave-uniform loop over its distinct bricks): one lane per brick claims or finds the
// bucket with a CAS and ORs in the occupancy bits of all its lanes, and every lane
// stores its row in its cell's slot. A cell set twice, inside the wave or by the
// atomicOr's old bits, is a repeated coordinate.
// keys: the sorted superblock-major cell keys (with perm; the coordinates are decoded
// from them), else sorted (with perm): the coordinates written in perm order here, for
// the probe (out-of-range rows too).
__global__ __launch_bounds__(256) void brick_insert_kernel(const int4* __restrict__ coords, int64_t n, Grid g,
                                                           const int32_t* __restrict__ perm,
                                                           const uint32_t* __restrict__ keys, BrickTable t,
                                                           int4* __restrict__ sorted, int32_t* __restrict__ status) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int lane = static_cast<int>(threadIdx.x & 63);
  bool act = i < n;
  int64_t row = i;
  int4 c = make_int4(0, 0, 0, 0);
  if (act && perm != nullptr) {
    const int32_t pp = perm[i];
    act = pp >= 0;
    row = pp;
    if (keys != nullptr) {
      if (act) c = g.sb_cell_decode(keys[i]);
    } else {
      c = coords[pp >= 0 ? pp : ~pp];
      sorted[i] = c;
    }
  } else if (act) {
    c = coords[row];
  }
  if (act && !g.inside(c.x, c.y, c.z, c.w)) {
    atomicOr(status, HI3D_MAP_RANGE);
    act = false;
  }
  const unsigned long long bk = act ? g.brick(c.x, c.y, c.z, c.w) : kEmptyBrick;
  const int cn = act ? g.corner(c.y, c.z, c.w) : 0;
  // group the wave's lanes by brick: `leader` is the first lane of this lane's brick,
  // `run` (at a leader) the lanes of its brick
  unsigned long long todo = __ballot(act);
  int leader = lane;
  unsigned long long run = 0;
  while (todo) {
    const int l = __ffsll(static_cast<long long>(todo)) - 1;
    const unsigned long long kl = shfl_u64(bk, l);
    const unsigned long long same = __ballot(act && bk == kl) & todo;
    if ((same >> lane) & 1ull) leader = l;
    if (lane == l) run = same;
    todo &= ~same;
  }
  unsigned long long cell[8];
#pragma unroll
  for (int b = 0; b < 8; ++b) cell[b] = __ballot(act && cn == b);
  unsigned long long h = 0;
  bool ok = true;
  if (act && leader == lane) {
    uint32_t bits = 0;
    bool dup = false;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const unsigned long long in_run = cell[b] & run;
      if (in_run) bits |= 1u << b;
      if (__popcll(in_run) > 1) dup = true;
    }
    h = g.brick_home(c.x, c.y >> 1, c.z >> 1, c.w >> 1, t.mask);
    const uint64_t step = brick_step(bk, t.mask);
    ok = false;
    for (uint64_t probe = 0; probe <= t.mask; ++probe) {
      const unsigned long long prev = atomicCAS(&t.words[h], kEmptyBrick, bk << 8);
      if (prev == kEmptyBrick || (prev >> 8) == bk) {
        ok = true;
        break;
      }
      h = (h + step) & t.mask;
    }
    if (ok) {
      const unsigned long long old = atomicOr(&t.words[h], static_cast<unsigned long long>(bits));
      if ((old & bits) || dup) atomicOr(status, HI3D_MAP_DUPLICATE);
    } else {
      atomicOr(status, HI3D_MAP_OVERFLOW);
    }
  }
  h = shfl_u64(h, leader);
  ok = __shfl(static_cast<int>(ok), leader, 64) != 0;
  if (act && ok) t.rows[h * 8 + cn] = static_cast<int32_t>(row);
}

// bucket of brick bk past its home h0 (whose key is already known to differ), or -1
__device__ __forceinline__ int64_t brick_find(const BrickTable& t, uint64_t h0, unsigned long long bk) {
  const uint64_t step = brick_step(bk, t.mask);
  uint64_t h = (h0 + step) & t.mask;
  for (uint64_t probe = 0; probe < t.mask; ++probe) {
    const unsigned long long w = t.words[h];
    if (w == kEmptyBrick) return -1;
    if ((w >> 8) == bk) return static_cast<int64_t>(h);
    h = (h + step) & t.mask;
  }
  return -1;
}

// One block: kProbeRows rows x kvol offsets, rows staged in LDS, each thread's cells
// kProbeBatch at a time: first every cell's bucket key (one independent load each), then
// the buckets' masks and rows (again independent loads).
__global__ __launch_bounds__(256) void brick_probe_kernel(const int4* __restrict__ coords, int64_t n, Grid g,
                                                          int ksize, const int32_t* __restrict__ perm, int per,
                                                          BrickTable t, int32_t* __restrict__ nbr,
                                                          int32_t* __restrict__ counts) {
  __shared__ int32_t cnt[kMaxKvol];
  __shared__ int4 sc[kProbeRows];
  __shared__ int32_t so[kProbeRows];
  const int kvol = ksize * ksize * ksize;
  const int half = ksize / 2;
  const int center = kvol / 2;
  const int64_t chunk = perm != nullptr ? static_cast<int64_t>(blockIdx.x % 8) * per + blockIdx.x / 8 : blockIdx.x;
  const int64_t row0 = chunk * kProbeRows;
  if (row0 >= n) return;  // the XCD order's spare blocks (before any barrier)
  const int rows = static_cast<int>(n - row0 < kProbeRows ? n - row0 : kProbeRows);
  for (int k = threadIdx.x; k < kvol; k += blockDim.x) cnt[k] = 0;
  if (threadIdx.x < rows) {
    int64_t o = row0 + threadIdx.x;
    if (perm != nullptr) {
      const int32_t p = perm[o];
      o = p >= 0 ? p : ~p;
    }
    so[threadIdx.x] = static_cast<int32_t>(o);
    sc[threadIdx.x] = coords[o];
  }
  __syncthreads();
  const int cells = rows * kvol;
  const int32_t absent = static_cast<int32_t>(n);
  for (int base = threadIdx.x; base < cells; base += blockDim.x * kProbeBatch) {
    unsigned long long bk[kProbeBatch], kv[kProbeBatch];
    uint64_t h[kProbeBatch];
    int cn[kProbeBatch];
    bool look[kProbeBatch];
#pragma unroll
    for (int u = 0; u < kProbeBatch; ++u) {
      const int j = base + u * blockDim.x;
      look[u] = false;
      bk[u] = kEmptyBrick;
      h[u] = 0;
      cn[u] = 0;
      if (j < cells) {
        const int r = j / kvol;
        const int k = j - r * kvol;
        const int4 c = sc[r];
        const int x = c.y + k / (ksize * ksize) - half;
        const int y = c.z + (k / ksize) % ksize - half;
        const int z = c.w + k % ksize - half;
        if (k != center && g.inside(c.x, x, y, z)) {
          look[u] = true;
          bk[u] = g.brick(c.x, x, y, z);
          h[u] = g.brick_home(c.x, x >> 1, y >> 1, z >> 1, t.mask);
          cn[u] = g.corner(x, y, z);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kProbeBatch; ++u) kv[u] = look[u] ? t.words[h[u]] : kEmptyBrick;
    int64_t hb[kProbeBatch];
    uint32_t m[kProbeBatch];
#pragma unroll
    for (int u = 0; u < kProbeBatch; ++u) {
      hb[u] = -1;
      m[u] = 0u;
      if (look[u] && kv[u] != kEmptyBrick) {
        if ((kv[u] >> 8) == bk[u]) {
          hb[u] = static_cast<int64_t>(h[u]);
          m[u] = static_cast<uint32_t>(kv[u] & 0xFFu);
        } else {
          hb[u] = brick_find(t, h[u], bk[u]);
          if (hb[u] >= 0) m[u] = static_cast<uint32_t>(t.words[hb[u]] & 0xFFu);
        }
      }
    }
    int32_t rv[kProbeBatch];
#pragma unroll
    for (int u = 0; u < kProbeBatch; ++u) rv[u] = ((m[u] >> cn[u]) & 1u) ? t.rows[hb[u] * 8 + cn[u]] : absent;
#pragma unroll
    for (int u = 0; u < kProbeBatch; ++u) {
      const int j = base + u * blockDim.x;
      if (j >= cells) continue;
      const int r = j / kvol;
      const int k = j - r * kvol;
      const int32_t o = so[r];
      const int32_t found = k == center ? o : rv[u];
      nbr[static_cast<int64_t>(o) * kvol + k] = found;
      if (found != absent) atomicAdd(&cnt[k], 1);
    }
  }
  __syncthreads();
  for (int k = threadIdx.x; k < kvol; k += blockDim.x)
    if (cnt[k]) atomicAdd(&counts[k], cnt[k]);
}

// The 3x3x3 probe: 8 lanes per row, lane l reading one of the 8 bricks that hold the
// row's 27 cells (bit 2 of l: the upper brick along x, bit 1: y, bit 0: z), so a row
// costs 8 bucket-word loads; each lane then resolves offsets l, l + 8, l + 16, l + 24
// from its row's 8 (mask, bucket) pairs (lane exchanges) and loads the rows of the
// present ones. A lane group carries kBrick3Per rows (32 rows apart), issuing their
// loads together, so kBrick3Per word loads and up to 4 kBrick3Per row loads per lane are
// in flight. The block's table rows are staged in LDS and written out whole. perm and
// per as in brick_probe_kernel, over blocks of kBrick3Rows rows.
constexpr int kBrick3Per = 4;
constexpr int kBrick3Rows = 32 * kBrick3Per;

// keys / sorted (with perm): as in brick_insert_kernel, so the coordinates load alongside
// perm.
// kPacked: buckets below 2^24, exchanged with their mask in one 32-bit lane move.
template <bool kPacked>
__global__ __launch_bounds__(256) void brick_probe3_kernel(const int4* __restrict__ coords, int64_t n, Grid g,
                                                           const int32_t* __restrict__ perm,
                                                           const uint32_t* __restrict__ keys,
                                                           const int4* __restrict__ sorted, int per, BrickTable t,
                                                           int32_t* __restrict__ nbr, int32_t* __restrict__ counts) {
  constexpr int P = kBrick3Per;
  __shared__ int32_t cnt[27];
  __shared__ int32_t stage[kBrick3Rows * 27];
  __shared__ int32_t srow[kBrick3Rows];
  const int64_t chunk = perm != nullptr ? static_cast<int64_t>(blockIdx.x % 8) * per + blockIdx.x / 8 : blockIdx.x;
  const int64_t row0 = chunk * kBrick3Rows;
  if (row0 >= n) return;  // the XCD order's spare blocks (before any barrier)
  if (threadIdx.x < 27) cnt[threadIdx.x] = 0;
  const int lane = threadIdx.x & 7;
  const int slot0 = threadIdx.x >> 3;  // the group's first row in the block; rows slot0 + 32 i
  const int group = static_cast<int>(threadIdx.x & 63) & ~7;  // the group's first lane in the wave
  const int64_t hx = (static_cast<int64_t>(g.sx) + 1) >> 1, hy = (static_cast<int64_t>(g.sy) + 1) >> 1,
                hz = (static_cast<int64_t>(g.sz) + 1) >> 1;
  bool valid[P];
  int32_t o[P];
  int4 c[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int64_t r = row0 + slot0 + 32 * i;
    valid[i] = r < n;
    int64_t oo = valid[i] ? r : 0;
    c[i] = make_int4(-1, 0, 0, 0);
    if (perm != nullptr && valid[i]) {
      const int32_t pp = perm[r];
      oo = pp >= 0 ? pp : ~pp;
      if (keys == nullptr)
        c[i] = sorted[r];
      else
        c[i] = pp >= 0 ? g.sb_cell_decode(keys[r]) : coords[oo];
    }
    o[i] = static_cast<int32_t>(oo);
  }
  if (perm == nullptr) {
#pragma unroll
    for (int i = 0; i < P; ++i)
      if (valid[i]) c[i] = coords[o[i]];
  }
  // the lane's brick: the lower (bit clear) or upper of the row's two neighbour bricks
  // along each axis, from lowest = (c >> 1) - 1 + (c & 1)
  uint32_t par[P];  // the row's coordinate parities (bit 2: x, 1: y, 0: z)
  uint64_t h[P];
  unsigned long long bk[P], w[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    par[i] = static_cast<uint32_t>(((c[i].y & 1) << 2) | ((c[i].z & 1) << 1) | (c[i].w & 1));
    const int64_t bx = (static_cast<int64_t>(c[i].y) >> 1) - 1 + (c[i].y & 1) + ((lane >> 2) & 1);
    const int64_t by = (static_cast<int64_t>(c[i].z) >> 1) - 1 + (c[i].z & 1) + ((lane >> 1) & 1);
    const int64_t bz = (static_cast<int64_t>(c[i].w) >> 1) - 1 + (c[i].w & 1) + (lane & 1);
    const bool in = valid[i] && static_cast<unsigned>(c[i].x) < static_cast<unsigned>(g.batch) && bx >= 0 &&
                    bx < hx && by >= 0 && by < hy && bz >= 0 && bz < hz;
    bk[i] = in ? g.brick_key(c[i].x, bx, by, bz) : kEmptyBrick;
    h[i] = in ? g.brick_home(c[i].x, bx, by, bz, t.mask) : 0ull;
  }
#pragma unroll
  for (int i = 0; i < P; ++i) w[i] = bk[i] != kEmptyBrick ? t.words[h[i]] : kEmptyBrick;
  // the lane's brick as (bucket << 8 | occupancy), 0 when absent
  uint64_t v[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    v[i] = 0;
    if (w[i] != kEmptyBrick) {
      if ((w[i] >> 8) == bk[i]) {
        v[i] = (h[i] << 8) | (w[i] & 0xFFu);
      } else {
        const int64_t f = brick_find(t, h[i], bk[i]);
        if (f >= 0) v[i] = (static_cast<uint64_t>(f) << 8) | (t.words[f] & 0xFFu);
      }
    }
  }
  // offsets l + 8 u: k = 9 (dx + 1) + 3 (dy + 1) + (dz + 1). Along an axis with parity p
  // the neighbour at d lies in brick (d + 2 - p) >> 1 of the two and has parity (p + d) & 1.
  int dx[4], dy[4], dz[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int kk = lane + 8 * u < 27 ? lane + 8 * u : 0;
    dx[u] = kk / 9 - 1;
    dy[u] = (kk / 3) % 3 - 1;
    dz[u] = kk % 3 - 1;
  }
  const int32_t absent = static_cast<int32_t>(n);
  int32_t found[P][4];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int px = (par[i] >> 2) & 1, py = (par[i] >> 1) & 1, pz = par[i] & 1;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int k = lane + 8 * u;
      const int j = (((dx[u] + 2 - px) >> 1) << 2) | (((dy[u] + 2 - py) >> 1) << 1) | ((dz[u] + 2 - pz) >> 1);
      const int cn = (((px + dx[u]) & 1) << 2) | (((py + dy[u]) & 1) << 1) | ((pz + dz[u]) & 1);
      const int src = group + j;
      uint64_t vj;
      if constexpr (kPacked) {
        vj = static_cast<uint32_t>(__shfl(static_cast<int>(static_cast<uint32_t>(v[i])), src, 64));
      } else {
        vj = shfl_u64(v[i], src);
      }
      found[i][u] = absent;
      if (valid[i] && k < 27 && k != 13 && ((vj >> cn) & 1u)) found[i][u] = t.rows[(vj >> 8) * 8 + cn];
    }
  }
  __syncthreads();  // cnt cleared
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int lr = slot0 + 32 * i;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int k = lane + 8 * u;
      if (k == 13) found[i][u] = o[i];
      const bool present = valid[i] && k < 27 && found[i][u] != absent;
      const unsigned long long ball = __ballot(present);
      if (k < 27) stage[lr * 27 + k] = found[i][u];
      // lane l of the wave's first group sums offset l + 8 u over the wave's 8 rows
      if ((threadIdx.x & 63) < 8 && k < 27) {
        const int c8 = __popcll(ball & (0x0101010101010101ull << lane));
        if (c8) atomicAdd(&cnt[k], c8);
      }
    }
    if (lane == 0) srow[lr] = valid[i] ? o[i] : -1;
  }
  __syncthreads();
  // whole rows: consecutive threads write consecutive entries of a row
  for (int e = threadIdx.x; e < kBrick3Rows * 27; e += blockDim.x) {
    const int rr = e / 27;
    const int32_t orow = srow[rr];
    if (orow >= 0) nbr[static_cast<int64_t>(orow) * 27 + (e - rr * 27)] = stage[e];
  }
  if (threadIdx.x < 27 && cnt[threadIdx.x]) atomicAdd(&counts[threadIdx.x], cnt[threadIdx.x]);
}

// Dense-grid variant for grids of at most kDenseMaxCells cells: one int32 cell per grid
// position holds its row (-1 empty). Every row stores its id in its cell (plain stores,
// the last of two equal coordinates wins) and the lookup flags a duplicate where a row's
// own cell holds another row; the lookups of a row read nine short z-runs of cells
// instead of random hash slots.
constexpr int64_t kDenseMaxCells = int64_t(1) << 31;
// cells before and after the grid in its buffer (the 12-byte z-runs read one past each
// end); 16 keep the grid 64-byte aligned
constexpr int64_t kDensePad = 16;

__global__ void dense_scatter_kernel(const int4* __restrict__ coords, int64_t n, Grid g, int32_t* __restrict__ cells,
                                     int32_t* __restrict__ status) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int4 c = coords[i];
  if (!g.inside(c.x, c.y, c.z, c.w)) {
    atomicOr(status, HI3D_MAP_RANGE);
    return;
  }
  cells[g.key(c.x, c.y, c.z, c.w)] = static_cast<int32_t>(i);
}

// Kept-grid path: rows are visited in cell order (a radix sort of the top kOrderBits bits
// of their cell keys), so the scatter, the lookups of neighbouring rows and the restore
// touch neighbouring cells.
// An out-of-range row is flagged, gets key 0 and the row id ~i (negative), and never
// touches the grid.
constexpr int kOrderBits = 16;

__global__ void cell_key_kernel(const int4* __restrict__ coords, int64_t n, Grid g, uint32_t* __restrict__ keys,
                                int32_t* __restrict__ rows, int32_t* __restrict__ status) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int4 c = coords[i];
  const bool in = g.inside(c.x, c.y, c.z, c.w);
  keys[i] = in ? static_cast<uint32_t>(g.key(c.x, c.y, c.z, c.w)) : 0u;
  rows[i] = in ? static_cast<int32_t>(i) : ~static_cast<int32_t>(i);
  if (!in) atomicOr(status, HI3D_MAP_RANGE);
}

// Brick-hash order: rows by superblock (8x8x8 cells), so consecutive rows insert into and
// probe the same runs of buckets; an out-of-range row is flagged, gets key 0 and the row
// id ~i. full: the whole superblock-major cell key (below 2^32: the insert and probe decode the
// coordinates from the sorted keys), else the superblock >> shift.
__global__ void superblock_key_kernel(const int4* __restrict__ coords, int64_t n, Grid g, int shift, bool full,
                                      uint32_t* __restrict__ keys, int32_t* __restrict__ rows,
                                      int32_t* __restrict__ status) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int4 c = coords[i];
  const bool in = g.inside(c.x, c.y, c.z, c.w);
  keys[i] = !in   ? 0u
            : full ? static_cast<uint32_t>(g.sb_cell_key(c.x, c.y, c.z, c.w))
                   : static_cast<uint32_t>(g.superblock(c.x, c.y >> 1, c.z >> 1, c.w >> 1) >> shift);
  rows[i] = in ? static_cast<int32_t>(i) : ~static_cast<int32_t>(i);
  if (!in) atomicOr(status, HI3D_MAP_RANGE);
}

// The sorted rows store their ids in their cells.
__global__ void sorted_scatter_kernel(const uint32_t* __restrict__ keys, const int32_t* __restrict__ rows, int64_t n,
                                      int32_t* __restrict__ cells) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n || rows[i] < 0) return;
  cells[keys[i]] = rows[i];
}

// Puts back the -1 of every cell the scatter may have claimed (out-of-range rows claim
// none; a duplicate's cell is its first row's).
__global__ void dense_restore_kernel(const int4* __restrict__ coords, int64_t n, Grid g, int32_t* __restrict__ cells) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int4 c = coords[i];
  if (g.inside(c.x, c.y, c.z, c.w)) cells[g.key(c.x, c.y, c.z, c.w)] = -1;
}

// Puts back the -1 of every cell the sorted rows claimed.
__global__ void sorted_restore_kernel(const uint32_t* __restrict__ keys, const int32_t* __restrict__ rows, int64_t n,
                                      int32_t* __restrict__ cells) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n || rows[i] < 0) return;
  cells[keys[i]] = -1;
}

// perm (optional): the block's rows are perm[row0 ..] instead of row0 .. (rows in cell
// order look up neighbouring cells; a negative entry p stands for the row ~p)
__global__ __launch_bounds__(256) void dense_lookup_kernel(const int4* __restrict__ coords, int64_t n, Grid g,
                                                           int ksize, const int32_t* __restrict__ cells,
                                                           const int32_t* __restrict__ perm,
                                                           int32_t* __restrict__ nbr, int32_t* __restrict__ counts,
                                                           int32_t* __restrict__ status) {
  __shared__ int32_t cnt[kMaxKvol];
  const int kvol = ksize * ksize * ksize;
  const int half = ksize / 2;
  const int center = kvol / 2;
  for (int k = threadIdx.x; k < kvol; k += blockDim.x) cnt[k] = 0;
  __syncthreads();
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kProbeRows;
  const int rows = static_cast<int>(n - row0 < kProbeRows ? n - row0 : kProbeRows);
  const int cells_n = rows * kvol;
  const int32_t absent = static_cast<int32_t>(n);
  for (int j = threadIdx.x; j < cells_n; j += blockDim.x) {
    const int r = j / kvol;
    const int k = j - r * kvol;
    int64_t o = row0 + r;
    if (perm != nullptr) {
      const int32_t p = perm[row0 + r];
      o = p >= 0 ? p : ~p;
    }
    int32_t found;
    if (k == center) {
      found = static_cast<int32_t>(o);
      const int4 c = coords[o];
      if (g.inside(c.x, c.y, c.z, c.w) && cells[g.key(c.x, c.y, c.z, c.w)] != found)
        atomicOr(status, HI3D_MAP_DUPLICATE);
    } else {
      const int4 c = coords[o];
      const int x = c.y + k / (ksize * ksize) - half;
      const int y = c.z + (k / ksize) % ksize - half;
      const int z = c.w + k % ksize - half;
      found = absent;
      if (g.inside(c.x, x, y, z)) {
        const int32_t v = cells[g.key(c.x, x, y, z)];
        if (v >= 0) found = v;
      }
    }
    nbr[o * kvol + k] = found;
    if (found != absent) atomicAdd(&cnt[k], 1);
  }
  __syncthreads();
  for (int k = threadIdx.x; k < kvol; k += blockDim.x)
    if (cnt[k]) atomicAdd(&counts[k], cnt[k]);
}

// The 3x3x3 lookup with one row per thread: the row's nine z-runs of three cells are
// nine independent 12-byte loads in flight together (a run starts one cell before the
// row's z, so the grid keeps a pad cell before and after; runs whose column lies outside
// the grid load at cell 0, and cells outside the grid are discarded), the counts
// are summed per wave with ballots, and the block's [256, 27] rows are staged in LDS so
// that the table is written in runs of whole rows. kPerm: the rows are perm[i] (rows in
// cell order, a negative entry p standing for the out-of-range row ~p), with their
// cells decoded from the sorted keys; the blocks then take the row chunks XCD by XCD
// (block b runs on XCD b % 8 and takes chunk (b % 8) * per + b / 8), so each XCD's L2
// sees a contiguous run of cells. Else the rows are i.
constexpr int kLookup3Rows = 256;
constexpr int kXcds = 8;
typedef int32_t ZRun __attribute__((ext_vector_type(3), aligned(4)));

template <bool kPerm>
__global__ __launch_bounds__(kLookup3Rows) void dense_lookup3_kernel(const int4* __restrict__ coords, int64_t n,
                                                                    Grid g, const int32_t* __restrict__ cells,
                                                                    const int32_t* __restrict__ perm,
                                                                    const uint32_t* __restrict__ skeys, int per,
                                                                    int32_t* __restrict__ nbr,
                                                                    int32_t* __restrict__ counts,
                                                                    int32_t* __restrict__ status) {
  __shared__ int32_t stage[kLookup3Rows * 27];
  __shared__ int32_t orow[kLookup3Rows];
  __shared__ int32_t cnt[27];
  const int t = threadIdx.x;
  if (t < 27) cnt[t] = 0;
  const int64_t chunk = kPerm ? static_cast<int64_t>(blockIdx.x % kXcds) * per + blockIdx.x / kXcds : blockIdx.x;
  const int64_t row0 = chunk * kLookup3Rows;
  if (row0 >= n) return;  // the XCD order's spare blocks (before any barrier)
  const int64_t i = row0 + t;
  const bool live = i < n;
  const int32_t absent = static_cast<int32_t>(n);
  int32_t o = 0;
  int4 c = make_int4(0, -2, -2, -2);  // a dead lane sees no cell inside the grid
  if (live) {
    if (kPerm) {
      const int32_t p = perm[i];
      if (p >= 0) {
        o = p;
        uint32_t key = skeys[i];
        c.w = static_cast<int>(key % static_cast<uint32_t>(g.sz));
        key /= static_cast<uint32_t>(g.sz);
        c.z = static_cast<int>(key % static_cast<uint32_t>(g.sy));
        key /= static_cast<uint32_t>(g.sy);
        c.y = static_cast<int>(key % static_cast<uint32_t>(g.sx));
        c.x = static_cast<int>(key / static_cast<uint32_t>(g.sx));
      } else {
        o = ~p;
        c = coords[o];
      }
    } else {
      o = static_cast<int32_t>(i);
      c = coords[o];
    }
    // An out-of-range row (flagged by the scatter or the key kernel) reads no cell: its
    // z-runs are checked per column only, so a z far outside the grid would otherwise
    // address cells far outside the buffer.
    if (!g.inside(c.x, c.y, c.z, c.w)) c = make_int4(0, -2, -2, -2);
  }
  orow[t] = o;
  const bool bin = static_cast<unsigned>(c.x) < static_cast<unsigned>(g.batch);
  bool okx[3], oky[3], okz[3];
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    okx[d] = bin && static_cast<unsigned>(c.y + d - 1) < static_cast<unsigned>(g.sx);
    oky[d] = static_cast<unsigned>(c.z + d - 1) < static_cast<unsigned>(g.sy);
    okz[d] = static_cast<unsigned>(c.w + d - 1) < static_cast<unsigned>(g.sz);
  }
  // key of the row's own cell; the neighbours are fixed strides away
  const int64_t base = ((static_cast<int64_t>(c.x) * g.sx + c.y) * g.sy + c.z) * g.sz + c.w;
  const int64_t sxs = static_cast<int64_t>(g.sy) * g.sz;
  int32_t f[27];
#pragma unroll
  for (int q = 0; q < 9; ++q) {
    const int dx = q / 3, dy = q % 3;
    const bool col = okx[dx] && oky[dy];
    const int64_t start = col ? base + (dx - 1) * sxs + (dy - 1) * g.sz - 1 : 0;
    const ZRun v = *reinterpret_cast<const ZRun*>(cells + start);
    f[q * 3 + 0] = col && okz[0] ? v.x : -1;
    f[q * 3 + 1] = col && okz[1] ? v.y : -1;
    f[q * 3 + 2] = col && okz[2] ? v.z : -1;
  }
  if (live && f[13] != o && okx[1] && oky[1] && okz[1]) atomicOr(status, HI3D_MAP_DUPLICATE);
  const int lane = t & 63;
  __syncthreads();  // cnt cleared
#pragma unroll
  for (int k = 0; k < 27; ++k) {
    int32_t v = f[k] >= 0 ? f[k] : absent;
    if (k == 13) v = live ? o : absent;
    const uint64_t hit = __ballot(v != absent);
    if (lane == 0 && hit != 0) atomicAdd(&cnt[k], static_cast<int32_t>(__popcll(hit)));
    stage[t * 27 + k] = v;
  }
  __syncthreads();
  const int rows = static_cast<int>(n - row0 < kLookup3Rows ? n - row0 : kLookup3Rows);
  if (kPerm) {
    for (int e = t; e < rows * 27; e += kLookup3Rows) {
      const int r = e / 27;
      nbr[static_cast<int64_t>(orow[r]) * 27 + (e - r * 27)] = stage[e];
    }
  } else {
    int32_t* dst = nbr + row0 * 27;
    for (int e = t; e < rows * 27; e += kLookup3Rows) dst[e] = stage[e];
  }
  if (t < 27 && cnt[t] != 0) atomicAdd(&counts[t], cnt[t]);
}

int64_t default_capacity(int64_t n) {
  int64_t cap = 64;
  while (cap < 2 * n) cap <<= 1;
  return cap;
}

// Default bucket count of the brick hash: one per voxel (a set whose voxels all sit in
// distinct bricks fills half of it; shells fill ~15 %).
int64_t brick_capacity(int64_t n) {
  int64_t cap = 64;
  while (cap < n) cap <<= 1;
  return cap;
}

// ------------------------------------------------------------------ pair lists --
constexpr int kPairRows = 256;  // rows per block (one per thread)

__global__ __launch_bounds__(256) void pair_count_kernel(const int32_t* __restrict__ nbr, int64_t n,
                                                         int kvol, int32_t* __restrict__ block_counts,
                                                         int64_t nblocks) {
  __shared__ int32_t wave_cnt[4];
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kPairRows + threadIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int k = 0; k < kvol; ++k) {
    bool present = i < n && nbr[i * kvol + (kvol - 1 - k)] != static_cast<int32_t>(n);
    uint64_t ballot = __ballot(present);
    if (lane == 0) wave_cnt[wave] = __popcll(ballot);
    __syncthreads();
    if (threadIdx.x == 0)
      block_counts[static_cast<int64_t>(k) * nblocks + blockIdx.x] =
          wave_cnt[0] + wave_cnt[1] + wave_cnt[2] + wave_cnt[3];
    __syncthreads();
  }
}

// One block per offset: exclusive scan of that offset's block counts (in place) and the
// offset's total.
__global__ __launch_bounds__(1024) void pair_scan_kernel(int32_t* __restrict__ block_counts,
                                                         int64_t nblocks,
                                                         int64_t* __restrict__ totals) {
  __shared__ int64_t wsum[16];
  __shared__ int64_t carry;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int32_t* row = block_counts + static_cast<int64_t>(blockIdx.x) * nblocks;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (int64_t base = 0; base < nblocks; base += 1024) {
    const int64_t idx = base + threadIdx.x;
    const int64_t v = idx < nblocks ? row[idx] : 0;
    int64_t x = v;  // inclusive scan within the wave, then across the 16 waves
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int64_t y = __shfl_up(x, d, 64);
      if (lane >= d) x += y;
    }
    if (lane == 63) wsum[w] = x;
    __syncthreads();
    int64_t off = 0, agg = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t p = wsum[i];
      off += i < w ? p : 0;
      agg += p;
    }
    if (idx < nblocks) row[idx] = static_cast<int32_t>(carry + off + x - v);
    __syncthreads();
    if (threadIdx.x == 0) carry += agg;
    __syncthreads();
  }
  if (threadIdx.x == 0) totals[blockIdx.x] = carry;
}

__global__ void pair_offsets_kernel(const int64_t* __restrict__ totals, int kvol,
                                    int64_t* __restrict__ offsets) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int64_t acc = 0;
  for (int k = 0; k < kvol; ++k) {
    offsets[k] = acc;
    acc += totals[k];
  }
  offsets[kvol] = acc;
}

__global__ __launch_bounds__(256) void pair_write_kernel(const int32_t* __restrict__ nbr, int64_t n,
                                                         int kvol,
                                                         const int32_t* __restrict__ block_offsets,
                                                         int64_t nblocks,
                                                         const int64_t* __restrict__ offsets,
                                                         int32_t* __restrict__ src,
                                                         int32_t* __restrict__ dst) {
  __shared__ int32_t wave_cnt[4];
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kPairRows + threadIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int k = 0; k < kvol; ++k) {
    int32_t j = i < n ? nbr[i * kvol + (kvol - 1 - k)] : static_cast<int32_t>(n);
    bool present = j != static_cast<int32_t>(n);
    uint64_t ballot = __ballot(present);
    if (lane == 0) wave_cnt[wave] = __popcll(ballot);
    __syncthreads();
    int before = 0;
    for (int w = 0; w < wave; ++w) before += wave_cnt[w];
    // rank of this lane among the present lanes below it in the wave
    int rank = __popcll(ballot & ((1ull << lane) - 1ull));
    if (present) {
      int64_t pos = offsets[k] + block_offsets[static_cast<int64_t>(k) * nblocks + blockIdx.x] + before + rank;
      src[pos] = static_cast<int32_t>(i);
      dst[pos] = j;
    }
    __syncthreads();
  }
}

// ------------------------------------------------ resampling (stride-f) structure --
// Factor (fx, fy, fz) per axis, F = fx fy fz slots per coarse cell (2, 2, 2 for the
// stride-2 pair). Sort key of fine row i: its coarse cell's packed code times F plus its
// slot ((x % fx) fy + y % fy) fz + z % fz, so the rows of one coarse cell sort together
// and two rows with the same coordinate sort next to each other. Coordinates outside
// [0, batch) x [0, sx) x [0, sy) x [0, sz) raise the range flag and take key 0 (the
// result is then discarded by the caller).
struct Factor {
  int32_t fx, fy, fz, hx, hy, hz;  // factors and coarse extents
  __device__ __forceinline__ uint64_t slots() const { return static_cast<uint64_t>(fx) * fy * fz; }
};

__global__ void factor_keys_kernel(const int4* __restrict__ coords, int64_t n, int32_t batch, int32_t sx, int32_t sy,
                                   int32_t sz, Factor f, unsigned long long* __restrict__ keys,
                                   int32_t* __restrict__ rows, int32_t* __restrict__ status) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int4 c = coords[i];
  const bool inside = c.x >= 0 && c.x < batch && c.y >= 0 && c.y < sx && c.z >= 0 && c.z < sy && c.w >= 0 && c.w < sz;
  if (!inside) {
    if (status) atomicOr(status, HI3D_MAP_RANGE);
    c = make_int4(0, 0, 0, 0);
  }
  const unsigned long long cell =
      ((static_cast<unsigned long long>(c.x) * f.hx + c.y / f.fx) * f.hy + c.z / f.fy) * f.hz + c.w / f.fz;
  const unsigned long long slot =
      (static_cast<unsigned long long>(c.y % f.fx) * f.fy + c.z % f.fy) * f.fz + c.w % f.fz;
  keys[i] = cell * f.slots() + slot;
  rows[i] = static_cast<int32_t>(i);
}

// heads[i] = 1 where sorted position i starts a coarse cell; equal neighbouring keys
// (same cell and slot) are a repeated coordinate
__global__ void run_heads_kernel(const unsigned long long* __restrict__ keys, int64_t n, uint64_t slots,
                                 int32_t* __restrict__ heads, int32_t* __restrict__ status) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const unsigned long long k = keys[i];
  const unsigned long long prev = i > 0 ? keys[i - 1] : ~k;
  heads[i] = (i == 0 || k / slots != prev / slots) ? 1 : 0;
  if (i > 0 && k == prev && status) atomicOr(status, HI3D_MAP_DUPLICATE);
}

// After the inclusive scan, ids[i] - 1 is the coarse row of sorted position i.
__global__ void coarse_emit_kernel(const unsigned long long* __restrict__ keys,
                                   const int32_t* __restrict__ rows,
                                   const int32_t* __restrict__ ids, int64_t n, Factor f,
                                   int4* __restrict__ low, int32_t* __restrict__ inverse,
                                   int32_t* __restrict__ counts, uint8_t* __restrict__ slot,
                                   int64_t* __restrict__ n_low) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint64_t slots = f.slots();
  const int32_t c = ids[i] - 1;
  const int32_t r = rows[i];
  inverse[r] = c;
  slot[r] = static_cast<uint8_t>(keys[i] % slots);
  const bool head = (i == 0) || keys[i] / slots != keys[i - 1] / slots;
  const bool tail = (i == n - 1) || keys[i] / slots != keys[i + 1] / slots;
  if (head) {
    unsigned long long k = keys[i] / slots;
    int4 l;
    l.w = static_cast<int>(k % f.hz);
    k /= f.hz;
    l.z = static_cast<int>(k % f.hy);
    k /= f.hy;
    l.y = static_cast<int>(k % f.hx);
    l.x = static_cast<int>(k / f.hx);
    low[c] = l;
    // run length = position of this run's tail - head + 1, written by the tail below
  }
  if (tail) {
    // find the head by walking back is O(run); instead counts are completed by a
    // second pass: store the tail position here, the head position at the head.
    counts[c] = static_cast<int32_t>(i);
  }
  if (i == n - 1) *n_low = static_cast<int64_t>(c) + 1;
}

__global__ void coarse_counts_kernel(const int32_t* __restrict__ ids, int64_t n,
                                     const unsigned long long* __restrict__ keys, uint64_t slots,
                                     int32_t* __restrict__ counts) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const bool head = (i == 0) || keys[i] / slots != keys[i - 1] / slots;
  if (head) {
    const int32_t c = ids[i] - 1;
    counts[c] = counts[c] - static_cast<int32_t>(i) + 1;  // tail - head + 1
  }
}

// down[inverse[i] * F + slot[i]] = i (the table arrives filled with the absent value n)
__global__ void factor_down_kernel(const int32_t* __restrict__ inverse, const uint8_t* __restrict__ slot, int64_t n,
                                   int32_t slots, int32_t* __restrict__ down) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  down[static_cast<int64_t>(inverse[i]) * slots + slot[i]] = static_cast<int32_t>(i);
}

// parent_table[o, k] = inverse[table[o, k]] for present entries, n_low for absent ones
__global__ void parent_table_kernel(const int32_t* __restrict__ table, int64_t total, int64_t n,
                                    const int32_t* __restrict__ inverse, int64_t n_low, int32_t* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int32_t t = table[i];
  out[i] = static_cast<uint64_t>(static_cast<uint32_t>(t)) < static_cast<uint64_t>(n) ? inverse[t]
                                                                                       : static_cast<int32_t>(n_low);
}

// out[i] = in[index[i]] for rows of rb bytes (a multiple of 16): one 16-byte chunk per
// thread
// Thread t copies chunks c, c + q, .. (G of them, q = cpr / G) of one row: one index
// load and G independent 16-byte loads in flight; consecutive threads still cover
// consecutive chunks in each of the G store steps.
template <int G>
__global__ void gather_rows_kernel(const char* __restrict__ in, int64_t n_in, int rb, const int32_t* __restrict__ index,
                                   int64_t n, char* __restrict__ out) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int q = (rb >> 4) / G;
  const int64_t row = t / q;
  if (row >= n) return;
  const int c = static_cast<int>(t - row * q);
  const int32_t src = index[row];
  const bool ok = static_cast<uint64_t>(static_cast<uint32_t>(src)) < static_cast<uint64_t>(n_in);
  uint4 v[G];
#pragma unroll
  for (int g = 0; g < G; ++g)
    v[g] = ok ? *reinterpret_cast<const uint4*>(in + static_cast<int64_t>(src) * rb + (c + g * q) * 16)
              : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
  for (int g = 0; g < G; ++g) *reinterpret_cast<uint4*>(out + row * rb + (c + g * q) * 16) = v[g];
}

__global__ void stride2_tables_kernel(const int32_t* __restrict__ inverse,
                                      const uint8_t* __restrict__ slot, int64_t n, int64_t n_low,
                                      int32_t* __restrict__ down, int32_t* __restrict__ up) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int32_t p = inverse[i];
  const int s = slot[i];
  if (down) down[static_cast<int64_t>(p) * 8 + s] = static_cast<int32_t>(i);
  if (up) {
    int4 a, b;
    a.x = s == 0 ? p : static_cast<int32_t>(n_low);
    a.y = s == 1 ? p : static_cast<int32_t>(n_low);
    a.z = s == 2 ? p : static_cast<int32_t>(n_low);
    a.w = s == 3 ? p : static_cast<int32_t>(n_low);
    b.x = s == 4 ? p : static_cast<int32_t>(n_low);
    b.y = s == 5 ? p : static_cast<int32_t>(n_low);
    b.z = s == 6 ? p : static_cast<int32_t>(n_low);
    b.w = s == 7 ? p : static_cast<int32_t>(n_low);
    reinterpret_cast<int4*>(up)[i * 2] = a;
    reinterpret_cast<int4*>(up)[i * 2 + 1] = b;
  }
}

// ---------------------------------------------------------------- child table --
// For child slot s and offset k: parent-neighbourhood offset holding the neighbour
// (pk) and the neighbour's own slot (ss); same construction as the reference's
// _child_offset_tables (sparse.py:46-61).
struct ChildTables {
  int8_t pk[8][27];
  int8_t ss[8][27];
};

ChildTables make_child_tables() {
  ChildTables t;
  for (int s = 0; s < 8; ++s) {
    int bits[3] = {(s >> 2) & 1, (s >> 1) & 1, s & 1};
    for (int k = 0; k < 27; ++k) {
      int d[3] = {k / 9 - 1, (k / 3) % 3 - 1, k % 3 - 1};
      int pd[3], cb[3];
      for (int a = 0; a < 3; ++a) {
        int v = bits[a] + d[a];  // in -1..2
        pd[a] = v >> 1;          // floor division
        cb[a] = v & 1;
      }
      t.pk[s][k] = static_cast<int8_t>((pd[0] + 1) * 9 + (pd[1] + 1) * 3 + (pd[2] + 1));
      t.ss[s][k] = static_cast<int8_t>(cb[0] * 4 + cb[1] * 2 + cb[2]);
    }
  }
  return t;
}

__global__ void mask_to_int_kernel(const uint8_t* __restrict__ mask, int64_t m, int32_t* __restrict__ out) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= m) return;
  out[i] = mask[i] ? 1 : 0;
}

// ids = exclusive scan of the mask: lookup[p*8+s] = child index (or C), plus parent/slot.
__global__ void child_index_kernel(const uint8_t* __restrict__ mask, const int32_t* __restrict__ excl,
                                   int64_t m, int32_t* __restrict__ lookup,
                                   int32_t* __restrict__ parent, int32_t* __restrict__ slot,
                                   int64_t* __restrict__ n_children) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= m) return;
  const int32_t total = excl[m - 1] + (mask[m - 1] ? 1 : 0);
  if (i == 0) *n_children = total;
  if (mask[i]) {
    const int32_t c = excl[i];
    lookup[i] = c;
    parent[c] = static_cast<int32_t>(i >> 3);
    slot[c] = static_cast<int32_t>(i & 7);
  } else {
    lookup[i] = total;
  }
  if (i < 8) lookup[m + i] = total;  // target of absent parents (row P)
}

__global__ void child_table_kernel(const int32_t* __restrict__ parent_table, const int32_t* __restrict__ lookup,
                                   const int32_t* __restrict__ parent, const int32_t* __restrict__ slot,
                                   const int64_t* __restrict__ n_children, int64_t cap, ChildTables t,
                                   int32_t* __restrict__ table) {
  int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t c = j / 27;
  if (c >= cap || c >= *n_children) return;
  const int k = static_cast<int>(j - c * 27);
  const int s = slot[c];
  const int32_t p = parent[c];
  const int32_t np = parent_table[static_cast<int64_t>(p) * 27 + t.pk[s][k]];
  table[j] = lookup[static_cast<int64_t>(np) * 8 + t.ss[s][k]];
}

// Hash table of hi3d_kmap_subm_noalloc: a device array of this library, one copy per GPU,
// held until the process ends. Host code never passes its name to a kernel (that is a
// host-side stand-in); it passes the address hipGetSymbolAddress returns for the
// current device.
static __device__ __align__(256) unsigned long long scratch[HI3D_KMAP_NOALLOC_BYTES / 8];

// Largest sets it takes: capacity (a power of two >= 2N) times 8 bytes (32-bit keys)
// or 8 + 4 bytes (64-bit keys) within the array.
constexpr int64_t kNoAllocMax32 = HI3D_KMAP_NOALLOC_BYTES / 8 / 2;
constexpr int64_t kNoAllocMax64 = HI3D_KMAP_NOALLOC_BYTES / 16 / 2;

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
char* g_scratch[kMaxDevices] = {};

// Address of the current device's copy of `scratch` (looked up once per device).
int scratch_address(char** out) {
  int dev = -1;
  HI3D_HIP_CHECK(hipGetDevice(&dev));
  HI3D_REQUIRE(dev >= 0 && dev < kMaxDevices, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    HI3D_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    HI3D_REQUIRE(p != nullptr && (reinterpret_cast<uintptr_t>(p) & 255) == 0, "scratch symbol has no usable address");
    g_scratch[dev] = static_cast<char*>(p);
  }
  *out = g_scratch[dev];
  return HI3D_OK;
}

}  // namespace
}  // namespace hi3d

using namespace hi3d;

extern "C" {

const char* hi3d_last_error(void) { return g_last_error.c_str(); }

const char* hi3d_version(void) { return "hi3d_amd 0.1 gfx950"; }

// Bytes of the cell-order sort that precedes a hash build: keys and rows (two slabs
// each) and the radix sort's counts.
static int64_t hash_order_bytes(int64_t n) {
  // keys, rows (two of each), the radix sort's temporaries, the coordinates in order
  return 4 * align_up(std::max<int64_t>(n, 1) * 4, 256) + align_up(radix::temp_bytes(std::max<int64_t>(n, 1)), 256) +
         align_up(std::max<int64_t>(n, 1) * 16, 256);
}

// Bytes of a brick table of `cap` buckets: key | mask words, then 8 rows per bucket.
static int64_t brick_table_bytes(int64_t cap) { return align_up(cap * 8, 256) + align_up(cap * 32, 256); }

// Brick tables above this size are built and probed in cell order (below it the table
// stays in the last-level cache and the sort costs more than it saves).
constexpr int64_t kBrickOrderMinBytes = int64_t(16) << 20;

int hi3d_kmap_workspace(int64_t n, int64_t capacity, int32_t key64, int64_t* bytes) {
  HI3D_REQUIRE(bytes != nullptr, "bytes_host is NULL");
  HI3D_REQUIRE(n >= 0, "n must be non-negative");
  (void)key64;  // bricks always use 64-bit keys
  int64_t cap = capacity > 0 ? capacity : brick_capacity(n);
  HI3D_REQUIRE((cap & (cap - 1)) == 0, "capacity must be a power of two");
  *bytes = brick_table_bytes(cap) + hash_order_bytes(n);
  return HI3D_OK;
}

// Argument checks shared by the hash-map entry points (clears counts and status).
static int kmap_subm_begin(const int32_t* coords, int64_t n, int32_t sx, int32_t sy, int32_t sz, int32_t batch_size,
                           int32_t ksize, int32_t* nbr, int32_t* counts, int32_t* status, hipStream_t stream) {
  HI3D_REQUIRE(n >= 0, "n must be non-negative");
  HI3D_REQUIRE(ksize >= 1 && ksize % 2 == 1 && ksize * ksize * ksize <= kMaxKvol,
               "ksize must be odd and at most 7, got %d", ksize);
  HI3D_REQUIRE(sx > 0 && sy > 0 && sz > 0 && batch_size > 0, "spatial_shape and batch_size must be positive");
  HI3D_REQUIRE(n < (int64_t(1) << 31) - 1, "at most 2^31-2 voxels");
  HI3D_REQUIRE(counts && status && (n == 0 || (coords && nbr)), "null pointer argument");
  const int kvol = ksize * ksize * ksize;
  launch_fill<int32_t>(counts, kvol, 0, stream);
  launch_fill<int32_t>(status, 1, 0, stream);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

// Voxel-slot hash build + probe over a table of `cap` slots at `table` (cap * 8 bytes of
// slots, then for 64-bit keys cap * 4 bytes of rows at the next 256-byte boundary), rows
// in input order: the allocation-free map's table, which fits its fixed array.
static int kmap_subm_hash(const int32_t* coords, int64_t n, Grid g, int32_t ksize, bool key64, int64_t cap,
                          char* table, int32_t* nbr, int32_t* counts, int32_t* status, hipStream_t stream) {
  const uint64_t mask = static_cast<uint64_t>(cap - 1);
  auto* slots = reinterpret_cast<unsigned long long*>(table);
  int32_t* vals = key64 ? reinterpret_cast<int32_t*>(table + align_up(cap * 8, 256)) : nullptr;
  const unsigned blocks = static_cast<unsigned>(ceil_div(n, 256));
  const int4* c4 = reinterpret_cast<const int4*>(coords);
  launch_fill<unsigned long long>(slots, cap, kEmpty, stream);
  const dim3 pgrid(static_cast<unsigned>(ceil_div(n, kProbeRows)));
  if (key64) {
    hipLaunchKernelGGL(insert64_kernel, dim3(blocks), dim3(256), 0, stream, c4, n, g, nullptr, slots, vals, mask,
                       status);
    hipLaunchKernelGGL(probe_kernel<true>, pgrid, dim3(256), 0, stream, c4, n, g, ksize, nullptr, 0, slots, vals, mask,
                       nbr, counts);
  } else {
    hipLaunchKernelGGL(insert32_kernel, dim3(blocks), dim3(256), 0, stream, c4, n, g, nullptr, slots, mask, status);
    hipLaunchKernelGGL(probe_kernel<false>, pgrid, dim3(256), 0, stream, c4, n, g, ksize, nullptr, 0, slots, nullptr,
                       mask, nbr, counts);
  }
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

// Brick-hash build + probe (hi3d_kmap_subm's map) over `cap` buckets at `ws`, with the
// cell-order sort when the table is large.
static int kmap_subm_brick(const int32_t* coords, int64_t n, Grid g, int32_t ksize, int64_t cap, char* ws,
                           int32_t* nbr, int32_t* counts, int32_t* status, hipStream_t stream) {
  BrickTable t;
  t.words = reinterpret_cast<unsigned long long*>(ws);
  t.rows = reinterpret_cast<int32_t*>(ws + align_up(cap * 8, 256));
  t.mask = static_cast<uint64_t>(cap - 1);
  char* order = ws + brick_table_bytes(cap);
  const unsigned blocks = static_cast<unsigned>(ceil_div(n, 256));
  const int4* c4 = reinterpret_cast<const int4*>(coords);
  const int32_t* perm = nullptr;
  int4* sorted = nullptr;
  const uint32_t* skeys = nullptr;
  int per = 0;
  int64_t probe_blocks = ceil_div(n, ksize == 3 ? kBrick3Rows : kProbeRows);
  if (brick_table_bytes(cap) > kBrickOrderMinBytes) {
    const int64_t slab = align_up(n * 4, 256);
    auto* k0 = reinterpret_cast<uint32_t*>(order);
    auto* k1 = reinterpret_cast<uint32_t*>(order + slab);
    auto* r0 = reinterpret_cast<int32_t*>(order + 2 * slab);
    auto* r1 = reinterpret_cast<int32_t*>(order + 3 * slab);
    const uint64_t q = static_cast<uint64_t>(g.batch) * ((((static_cast<uint64_t>(g.sx) + 1) / 2) + 3) >> 2) *
                       ((((static_cast<uint64_t>(g.sy) + 1) / 2) + 3) >> 2) *
                       ((((static_cast<uint64_t>(g.sz) + 1) / 2) + 3) >> 2);
    int key_bits = 1;
    while (key_bits < 64 && (uint64_t(1) << key_bits) < q) ++key_bits;
    // whole cell keys when they fit 32 bits (sorted by their top 24), else the superblock's
    // top 32 bits
    const bool full = key_bits + 9 <= 32;
    const int shift = full || key_bits <= 32 ? 0 : key_bits - 32;
    const int kb = full ? key_bits + 9 : key_bits - shift;
    hipLaunchKernelGGL(superblock_key_kernel, dim3(blocks), dim3(256), 0, stream, c4, n, g, shift, full, k0, r0,
                       status);
    HI3D_HIP_CHECK(radix::sort_pairs(order + 4 * slab, radix::temp_bytes(n), k0, k1, r0, r1, n,
                                     kb > 24 ? kb - 24 : 0, kb, stream));
    perm = r0;
    if (full)
      skeys = k0;
    else
      sorted = reinterpret_cast<int4*>(order + 4 * slab + align_up(radix::temp_bytes(n), 256));
    per = static_cast<int>(ceil_div(probe_blocks, kXcds));
    probe_blocks = static_cast<int64_t>(per) * kXcds;
  }
  launch_fill<unsigned long long>(t.words, cap, kEmptyBrick, stream);
  hipLaunchKernelGGL(brick_insert_kernel, dim3(blocks), dim3(256), 0, stream, c4, n, g, perm, skeys, t, sorted,
                     status);
  if (ksize == 3 && cap <= (int64_t(1) << 24))
    hipLaunchKernelGGL(brick_probe3_kernel<true>, dim3(static_cast<unsigned>(probe_blocks)), dim3(256), 0, stream, c4,
                       n, g, perm, skeys, sorted, per, t, nbr, counts);
  else if (ksize == 3)
    hipLaunchKernelGGL(brick_probe3_kernel<false>, dim3(static_cast<unsigned>(probe_blocks)), dim3(256), 0, stream, c4,
                       n, g, perm, skeys, sorted, per, t, nbr, counts);
  else
    hipLaunchKernelGGL(brick_probe_kernel, dim3(static_cast<unsigned>(probe_blocks)), dim3(256), 0, stream, c4, n, g,
                       ksize, perm, per, t, nbr, counts);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

int hi3d_kmap_subm(const int32_t* coords, int64_t n, int32_t sx, int32_t sy, int32_t sz,
                   int32_t batch_size, int32_t ksize, int64_t capacity, void* workspace,
                   int64_t workspace_bytes, int32_t* nbr, int32_t* counts, int32_t* status,
                   void* stream_) {
  hipStream_t stream = as_stream(stream_);
  int rc = kmap_subm_begin(coords, n, sx, sy, sz, batch_size, ksize, nbr, counts, status, stream);
  if (rc != HI3D_OK || n == 0) return rc;
  HI3D_REQUIRE(workspace != nullptr, "null pointer argument");
  const int64_t cap = capacity > 0 ? capacity : brick_capacity(n);
  const double bricks = static_cast<double>(batch_size) * ((sx + 1) / 2) * ((sy + 1) / 2) * ((sz + 1) / 2);
  HI3D_REQUIRE(bricks < 7.2e16, "grid of %.3g 2x2x2 bricks exceeds the hash's 2^56 brick keys", bricks);
  int64_t need = 0;
  rc = hi3d_kmap_workspace(n, cap, 1, &need);
  if (rc != HI3D_OK) return rc;
  HI3D_REQUIRE(workspace_bytes >= need, "workspace too small: %lld < %lld bytes",
               static_cast<long long>(workspace_bytes), static_cast<long long>(need));
  return kmap_subm_brick(coords, n, Grid{sx, sy, sz, batch_size}, ksize, cap, static_cast<char*>(workspace), nbr,
                         counts, status, stream);
}

// The same map with the hash table in `scratch`, a device array of this library (no
// allocation, no workspace). Every call on a GPU reuses that GPU's copy: calls that
// overlap on one GPU (two streams, two host threads) race on it.
int hi3d_kmap_subm_noalloc(const int32_t* coords, int64_t n, int32_t sx, int32_t sy, int32_t sz, int32_t batch_size,
                           int32_t ksize, int32_t* nbr, int32_t* counts, int32_t* status, void* stream_) {
  hipStream_t stream = as_stream(stream_);
  int rc = kmap_subm_begin(coords, n, sx, sy, sz, batch_size, ksize, nbr, counts, status, stream);
  if (rc != HI3D_OK || n == 0) return rc;
  const uint64_t space = static_cast<uint64_t>(batch_size) * sx * sy * sz;
  const bool key64 = space >= 0xFFFFFFFFull;
  const int64_t cap = default_capacity(n);
  const int64_t need = key64 ? align_up(cap * 8, 256) + cap * 4 : cap * 8;  // slots (+ rows)
  HI3D_REQUIRE(need <= HI3D_KMAP_NOALLOC_BYTES,
               "%lld voxels need a %lld-byte hash table; the allocation-free map holds at most %lld bytes (%s keys: up "
               "to %lld voxels)",
               static_cast<long long>(n), static_cast<long long>(need), static_cast<long long>(HI3D_KMAP_NOALLOC_BYTES),
               key64 ? "64-bit" : "32-bit", static_cast<long long>(key64 ? kNoAllocMax64 : kNoAllocMax32));
  char* table = nullptr;
  rc = scratch_address(&table);
  if (rc != HI3D_OK) return rc;
  return kmap_subm_hash(coords, n, Grid{sx, sy, sz, batch_size}, ksize, key64, cap, table, nbr, counts, status,
                        stream);
}

int hi3d_kmap_dense_workspace(int32_t batch_size, int32_t sx, int32_t sy, int32_t sz, int64_t* bytes) {
  HI3D_REQUIRE(bytes != nullptr, "bytes_host is NULL");
  HI3D_REQUIRE(sx > 0 && sy > 0 && sz > 0 && batch_size > 0, "spatial_shape and batch_size must be positive");
  const int64_t cells = static_cast<int64_t>(batch_size) * sx * sy * sz;
  HI3D_REQUIRE(cells <= kDenseMaxCells, "dense map grid of %lld cells exceeds 2^31", static_cast<long long>(cells));
  *bytes = align_up((cells + 2 * kDensePad) * 4, 256);
  return HI3D_OK;
}

int hi3d_kmap_dense_order_workspace(int64_t n, int64_t* bytes) {
  HI3D_REQUIRE(bytes != nullptr, "bytes_host is NULL");
  HI3D_REQUIRE(n >= 0 && n < (int64_t(1) << 31) - 1, "bad voxel count");
  *bytes = 4 * align_up(n * 4, 256) + radix::temp_bytes(n);
  return HI3D_OK;
}

}  // extern "C"

namespace {

void launch_dense_lookup(const int4* c4, int64_t n, Grid g, int ksize, const int32_t* cells, const int32_t* perm,
                         const uint32_t* skeys, int32_t* nbr, int32_t* counts, int32_t* status, hipStream_t stream) {
  if (ksize == 3) {
    const int64_t chunks = ceil_div(n, kLookup3Rows);
    if (perm != nullptr) {
      const int64_t per = ceil_div(chunks, kXcds);
      hipLaunchKernelGGL(dense_lookup3_kernel<true>, dim3(static_cast<unsigned>(per * kXcds)), dim3(kLookup3Rows), 0,
                         stream, c4, n, g, cells, perm, skeys, static_cast<int>(per), nbr, counts, status);
    } else {
      hipLaunchKernelGGL(dense_lookup3_kernel<false>, dim3(static_cast<unsigned>(chunks)), dim3(kLookup3Rows), 0,
                         stream, c4, n, g, cells, perm, skeys, 0, nbr, counts, status);
    }
    return;
  }
  hipLaunchKernelGGL(dense_lookup_kernel, dim3(static_cast<unsigned>(ceil_div(n, kProbeRows))), dim3(256), 0, stream,
                     c4, n, g, ksize, cells, perm, nbr, counts, status);
}

// kept: the grid arrives with every cell -1 and is left that way (the scatter's cells
// are put back after the lookup), instead of being cleared whole on entry. order (kept
// only, may be NULL): workspace for visiting the rows in cell order.
int kmap_subm_dense(const int32_t* coords, int64_t n, int32_t sx, int32_t sy, int32_t sz, int32_t batch_size,
                    int32_t ksize, void* workspace, int64_t workspace_bytes, int32_t* nbr, int32_t* counts,
                    int32_t* status, void* stream_, bool kept, void* order = nullptr, int64_t order_bytes = 0) {
  hipStream_t stream = as_stream(stream_);
  HI3D_REQUIRE(n >= 0, "n must be non-negative");
  HI3D_REQUIRE(ksize >= 1 && ksize % 2 == 1 && ksize * ksize * ksize <= kMaxKvol,
               "ksize must be odd and at most 7, got %d", ksize);
  HI3D_REQUIRE(n < (int64_t(1) << 31) - 1, "at most 2^31-2 voxels");
  int64_t need = 0;
  int rc = hi3d_kmap_dense_workspace(batch_size, sx, sy, sz, &need);
  if (rc != HI3D_OK) return rc;
  HI3D_REQUIRE(counts && status && (n == 0 || (coords && nbr && workspace)), "null pointer argument");
  const int kvol = ksize * ksize * ksize;
  launch_fill<int32_t>(counts, kvol, 0, stream);
  launch_fill<int32_t>(status, 1, 0, stream);
  if (n == 0) {
    HI3D_LAUNCH_CHECK();
    return HI3D_OK;
  }
  HI3D_REQUIRE(workspace_bytes >= need, "workspace too small: %lld < %lld bytes",
               static_cast<long long>(workspace_bytes), static_cast<long long>(need));
  Grid g{sx, sy, sz, batch_size};
  auto* cells = static_cast<int32_t*>(workspace) + kDensePad;
  if (!kept) {
    // clear the grid with 16-byte stores (the workspace is 256-byte aligned)
    const int64_t ncells = static_cast<int64_t>(batch_size) * sx * sy * sz;
    launch_fill<int4>(reinterpret_cast<int4*>(cells), ncells / 4, make_int4(-1, -1, -1, -1), stream);
    launch_fill<int32_t>(cells + (ncells & ~int64_t(3)), ncells & 3, -1, stream);
  }
  const int4* c4 = reinterpret_cast<const int4*>(coords);
  if (kept && order != nullptr) {
    int64_t order_need = 0;
    rc = hi3d_kmap_dense_order_workspace(n, &order_need);
    if (rc != HI3D_OK) return rc;
    HI3D_REQUIRE(order_bytes >= order_need, "order workspace too small: %lld < %lld bytes",
                 static_cast<long long>(order_bytes), static_cast<long long>(order_need));
    const int64_t slab = align_up(n * 4, 256);
    char* w = static_cast<char*>(order);
    auto* k0 = reinterpret_cast<uint32_t*>(w);
    auto* k1 = reinterpret_cast<uint32_t*>(w + slab);
    auto* r0 = reinterpret_cast<int32_t*>(w + 2 * slab);
    auto* r1 = reinterpret_cast<int32_t*>(w + 3 * slab);
    void* temp = w + 4 * slab;
    const int64_t temp_bytes = order_bytes - 4 * slab;
    const dim3 grid1(static_cast<unsigned>(ceil_div(n, 256)));
    hipLaunchKernelGGL(cell_key_kernel, grid1, dim3(256), 0, stream, c4, n, g, k0, r0, status);
    const int64_t ncells = static_cast<int64_t>(batch_size) * sx * sy * sz;
    int key_bits = 1;
    while (key_bits < 32 && (int64_t(1) << key_bits) < ncells) ++key_bits;
    // two radix passes over the key's top 16 bits (batch, x, y bands) give the lookups
    // their locality; the keys move whole, so every row still knows its cell
    const int low_bit = key_bits > kOrderBits ? key_bits - kOrderBits : 0;
    HI3D_HIP_CHECK(radix::sort_pairs(temp, temp_bytes, k0, k1, r0, r1, n, low_bit, key_bits, stream));
    hipLaunchKernelGGL(sorted_scatter_kernel, grid1, dim3(256), 0, stream, k0, r0, n, cells);
    launch_dense_lookup(c4, n, g, ksize, cells, r0, k0, nbr, counts, status, stream);
    hipLaunchKernelGGL(sorted_restore_kernel, grid1, dim3(256), 0, stream, k0, r0, n, cells);
    HI3D_LAUNCH_CHECK();
    return HI3D_OK;
  }
  hipLaunchKernelGGL(dense_scatter_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0, stream, c4, n,
                     g, cells, status);
  launch_dense_lookup(c4, n, g, ksize, cells, nullptr, nullptr, nbr, counts, status, stream);
  if (kept)
    hipLaunchKernelGGL(dense_restore_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0, stream, c4,
                       n, g, cells);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

}  // namespace

extern "C" {

int hi3d_kmap_subm_dense(const int32_t* coords, int64_t n, int32_t sx, int32_t sy, int32_t sz, int32_t batch_size,
                         int32_t ksize, void* workspace, int64_t workspace_bytes, int32_t* nbr, int32_t* counts,
                         int32_t* status, void* stream) {
  return kmap_subm_dense(coords, n, sx, sy, sz, batch_size, ksize, workspace, workspace_bytes, nbr, counts, status,
                         stream, false);
}

int hi3d_kmap_subm_dense_kept(const int32_t* coords, int64_t n, int32_t sx, int32_t sy, int32_t sz,
                              int32_t batch_size, int32_t ksize, void* grid, int64_t grid_bytes, void* order,
                              int64_t order_bytes, int32_t* nbr, int32_t* counts, int32_t* status, void* stream) {
  return kmap_subm_dense(coords, n, sx, sy, sz, batch_size, ksize, grid, grid_bytes, nbr, counts, status, stream,
                         true, order, order_bytes);
}

int hi3d_kmap_pairs_workspace(int64_t n, int32_t kvol, int64_t* bytes) {
  HI3D_REQUIRE(bytes != nullptr, "bytes_host is NULL");
  HI3D_REQUIRE(n >= 0 && kvol > 0, "bad sizes");
  const int64_t nblocks = std::max<int64_t>(1, ceil_div(n, kPairRows));
  *bytes = align_up(nblocks * kvol * 4, 256) + align_up(static_cast<int64_t>(kvol) * 8, 256);
  return HI3D_OK;
}

int hi3d_kmap_pairs(const int32_t* nbr, int64_t n, int32_t kvol, void* workspace, int64_t workspace_bytes,
                    int32_t* src, int32_t* dst, int64_t* offsets, void* stream_) {
  hipStream_t stream = as_stream(stream_);
  int64_t need = 0;
  int rc = hi3d_kmap_pairs_workspace(n, kvol, &need);
  if (rc != HI3D_OK) return rc;
  HI3D_REQUIRE(offsets != nullptr, "offsets_dev is NULL");
  if (n == 0) {
    launch_fill<int64_t>(offsets, kvol + 1, 0, stream);
    HI3D_LAUNCH_CHECK();
    return HI3D_OK;
  }
  HI3D_REQUIRE(nbr && src && dst && workspace, "null pointer argument");
  HI3D_REQUIRE(workspace_bytes >= need, "workspace too small");
  const int64_t nblocks = ceil_div(n, kPairRows);
  Workspace ws(workspace, workspace_bytes);
  int32_t* block_counts = ws.take<int32_t>(nblocks * kvol);
  int64_t* totals = ws.take<int64_t>(kvol);
  hipLaunchKernelGGL(pair_count_kernel, dim3(static_cast<unsigned>(nblocks)), dim3(256), 0, stream, nbr, n, kvol,
                     block_counts, nblocks);
  hipLaunchKernelGGL(pair_scan_kernel, dim3(kvol), dim3(1024), 0, stream, block_counts, nblocks, totals);
  hipLaunchKernelGGL(pair_offsets_kernel, dim3(1), dim3(64), 0, stream, totals, kvol, offsets);
  hipLaunchKernelGGL(pair_write_kernel, dim3(static_cast<unsigned>(nblocks)), dim3(256), 0, stream, nbr, n, kvol,
                     block_counts, nblocks, offsets, src, dst);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

int hi3d_downsample_workspace(int64_t n, int64_t* bytes) {
  HI3D_REQUIRE(bytes != nullptr, "bytes_host is NULL");
  HI3D_REQUIRE(n >= 0 && n < (int64_t(1) << 31) - 1, "bad n");
  const int64_t m = std::max<int64_t>(n, 1);
  *bytes = 2 * align_up(m * 8, 256) + 3 * align_up(m * 4, 256) + radix::temp_bytes(m) + 256;
  return HI3D_OK;
}

// The coarse structure of a resampling by factor (fx, fy, fz) (workspace as
// hi3d_downsample_workspace).
static int resample_structure(const int32_t* coords, int64_t n, int32_t sx, int32_t sy, int32_t sz,
                              int32_t batch_size, int32_t fx, int32_t fy, int32_t fz, void* workspace,
                              int64_t workspace_bytes, int32_t* low, int32_t* inverse, int32_t* counts,
                              uint8_t* slot, int64_t* n_low, int32_t* status, hipStream_t stream) {
  int64_t need = 0;
  int rc = hi3d_downsample_workspace(n, &need);
  if (rc != HI3D_OK) return rc;
  HI3D_REQUIRE(n_low != nullptr, "n_low_dev is NULL");
  HI3D_REQUIRE(fx > 0 && fy > 0 && fz > 0 && static_cast<int64_t>(fx) * fy * fz <= 256,
               "factors must be positive with a product of at most 256, got (%d, %d, %d)", fx, fy, fz);
  if (status) launch_fill<int32_t>(status, 1, 0, stream);
  if (n == 0) {
    launch_fill<int64_t>(n_low, 1, 0, stream);
    HI3D_LAUNCH_CHECK();
    return HI3D_OK;
  }
  HI3D_REQUIRE(coords && low && inverse && counts && slot && workspace, "null pointer argument");
  HI3D_REQUIRE(workspace_bytes >= need, "workspace too small");
  HI3D_REQUIRE(sx > 0 && sy > 0 && sz > 0 && batch_size > 0, "spatial_shape and batch_size must be positive");
  const Factor f{fx, fy, fz, (sx + fx - 1) / fx, (sy + fy - 1) / fy, (sz + fz - 1) / fz};
  const uint64_t slots = static_cast<uint64_t>(fx) * fy * fz;
  Workspace ws(workspace, workspace_bytes);
  auto* k0 = ws.take<unsigned long long>(n);
  auto* k1 = ws.take<unsigned long long>(n);
  auto* r0 = ws.take<int32_t>(n);
  auto* r1 = ws.take<int32_t>(n);
  auto* ids = ws.take<int32_t>(n);
  const int64_t temp_bytes = radix::temp_bytes(n);
  void* temp = ws.take<char>(temp_bytes);
  const unsigned blocks = static_cast<unsigned>(ceil_div(n, 256));
  const int4* c4 = reinterpret_cast<const int4*>(coords);
  const double space_d = static_cast<double>(batch_size) * f.hx * f.hy * f.hz * static_cast<double>(slots);
  HI3D_REQUIRE(space_d < 4.0e18, "grid too large for 64-bit keys");
  const uint64_t space = static_cast<uint64_t>(batch_size) * f.hx * f.hy * f.hz * slots;  // cells x slots
  hipLaunchKernelGGL(factor_keys_kernel, dim3(blocks), dim3(256), 0, stream, c4, n, batch_size, sx, sy, sz, f, k0, r0,
                     status);
  int end_bit = 1;
  while (end_bit < 64 && (1ull << end_bit) < space) ++end_bit;
  unsigned long long* ka = k0;
  unsigned long long* kalt = k1;
  int32_t* ra = r0;
  int32_t* ralt = r1;
  HI3D_HIP_CHECK(radix::sort_pairs(temp, temp_bytes, ka, kalt, ra, ralt, n, 0, end_bit, stream));
  const unsigned long long* sk = ka;
  const int32_t* sr = ra;
  hipLaunchKernelGGL(run_heads_kernel, dim3(blocks), dim3(256), 0, stream, sk, n, slots, ids, status);
  HI3D_HIP_CHECK(radix::scan(temp, temp_bytes, ids, ids, n, true, stream));
  hipLaunchKernelGGL(coarse_emit_kernel, dim3(blocks), dim3(256), 0, stream, sk, sr, ids, n, f,
                     reinterpret_cast<int4*>(low), inverse, counts, slot, n_low);
  hipLaunchKernelGGL(coarse_counts_kernel, dim3(blocks), dim3(256), 0, stream, ids, n, sk, slots, counts);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

int hi3d_downsample_structure(const int32_t* coords, int64_t n, int32_t sx, int32_t sy, int32_t sz,
                              int32_t batch_size, void* workspace, int64_t workspace_bytes, int32_t* low,
                              int32_t* inverse, int32_t* counts, uint8_t* slot, int64_t* n_low, int32_t* status,
                              void* stream) {
  return resample_structure(coords, n, sx, sy, sz, batch_size, 2, 2, 2, workspace, workspace_bytes, low, inverse,
                            counts, slot, n_low, status, as_stream(stream));
}

int hi3d_resample_structure(const int32_t* coords, int64_t n, int32_t sx, int32_t sy, int32_t sz, int32_t batch_size,
                            int32_t fx, int32_t fy, int32_t fz, void* workspace, int64_t workspace_bytes, int32_t* low,
                            int32_t* inverse, int32_t* counts, uint8_t* slot, int64_t* n_low, int32_t* status,
                            void* stream) {
  return resample_structure(coords, n, sx, sy, sz, batch_size, fx, fy, fz, workspace, workspace_bytes, low, inverse,
                            counts, slot, n_low, status, as_stream(stream));
}

int hi3d_resample_down_table(const int32_t* inverse, const uint8_t* slot, int64_t n, int64_t n_low, int32_t slots,
                             int32_t* down, void* stream_) {
  hipStream_t stream = as_stream(stream_);
  HI3D_REQUIRE(n >= 0 && n_low >= 0 && slots >= 1 && slots <= 256, "bad sizes");
  if (n_low == 0) return HI3D_OK;
  HI3D_REQUIRE(down != nullptr, "null pointer argument");
  launch_fill<int32_t>(down, n_low * slots, static_cast<int32_t>(n), stream);
  if (n > 0) {
    HI3D_REQUIRE(inverse && slot, "null pointer argument");
    hipLaunchKernelGGL(factor_down_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0, stream,
                       inverse, slot, n, slots, down);
  }
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

int hi3d_stride2_tables(const int32_t* inverse, const uint8_t* slot, int64_t n, int64_t n_low, int32_t* down,
                        int32_t* up, void* stream_) {
  hipStream_t stream = as_stream(stream_);
  HI3D_REQUIRE(n >= 0 && n_low >= 0, "bad sizes");
  if (n == 0) return HI3D_OK;
  HI3D_REQUIRE(inverse && slot, "null pointer argument");
  if (down) launch_fill<int32_t>(down, n_low * 8, static_cast<int32_t>(n), stream);
  hipLaunchKernelGGL(stride2_tables_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0, stream,
                     inverse, slot, n, n_low, down, up);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

int hi3d_parent_table(const int32_t* table, int64_t n, int32_t kvol, const int32_t* inverse, int64_t n_low,
                      int32_t* out, void* stream_) {
  hipStream_t stream = as_stream(stream_);
  HI3D_REQUIRE(n >= 0 && n_low >= 0 && n_low < (int64_t(1) << 31) - 1 && kvol >= 1 && kvol <= 1024, "bad sizes");
  if (n == 0) return HI3D_OK;
  HI3D_REQUIRE(table && inverse && out, "null pointer argument");
  const int64_t total = n * kvol;
  hipLaunchKernelGGL(parent_table_kernel, dim3(static_cast<unsigned>(ceil_div(total, 256))), dim3(256), 0, stream,
                     table, total, n, inverse, n_low, out);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

int hi3d_gather_rows(const void* in, int64_t n_in, int32_t row_bytes, const int32_t* index, int64_t n, void* out,
                     void* stream_) {
  hipStream_t stream = as_stream(stream_);
  HI3D_REQUIRE(row_bytes > 0 && row_bytes % 16 == 0, "row bytes must be a positive multiple of 16, got %d", row_bytes);
  HI3D_REQUIRE(n >= 0 && n_in >= 0, "bad sizes");
  if (n == 0) return HI3D_OK;
  HI3D_REQUIRE(in && index && out, "null pointer argument");
  HI3D_REQUIRE(((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15) == 0,
               "rows must be 16-byte aligned");
  const int cpr = row_bytes / 16;
  if (cpr % 4 == 0) {
    const int64_t total = n * (cpr / 4);
    hipLaunchKernelGGL(gather_rows_kernel<4>, dim3(static_cast<unsigned>(ceil_div(total, 256))), dim3(256), 0, stream,
                       static_cast<const char*>(in), n_in, row_bytes, index, n, static_cast<char*>(out));
  } else {
    const int64_t total = n * cpr;
    hipLaunchKernelGGL(gather_rows_kernel<1>, dim3(static_cast<unsigned>(ceil_div(total, 256))), dim3(256), 0, stream,
                       static_cast<const char*>(in), n_in, row_bytes, index, n, static_cast<char*>(out));
  }
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

int hi3d_child_table_workspace(int64_t n_parents, int64_t* bytes) {
  HI3D_REQUIRE(bytes != nullptr, "bytes_host is NULL");
  HI3D_REQUIRE(n_parents >= 0 && n_parents * 8 < (int64_t(1) << 31) - 16, "bad n_parents");
  const int64_t m = std::max<int64_t>(n_parents * 8, 1);
  *bytes = 2 * align_up(m * 4, 256) + align_up((m + 8) * 4, 256) + radix::temp_bytes(m);
  return HI3D_OK;
}

int hi3d_child_neighbour_table(const int32_t* parent_table, const uint8_t* mask, int64_t n_parents,
                               void* workspace, int64_t workspace_bytes, int32_t* table, int32_t* parent,
                               int32_t* slot, int64_t* n_children, void* stream_) {
  hipStream_t stream = as_stream(stream_);
  int64_t need = 0;
  int rc = hi3d_child_table_workspace(n_parents, &need);
  if (rc != HI3D_OK) return rc;
  HI3D_REQUIRE(n_children != nullptr, "n_children_dev is NULL");
  if (n_parents == 0) {
    launch_fill<int64_t>(n_children, 1, 0, stream);
    HI3D_LAUNCH_CHECK();
    return HI3D_OK;
  }
  HI3D_REQUIRE(parent_table && mask && table && parent && slot && workspace, "null pointer argument");
  HI3D_REQUIRE(workspace_bytes >= need, "workspace too small");
  const int64_t m = n_parents * 8;
  Workspace ws(workspace, workspace_bytes);
  int32_t* flags = ws.take<int32_t>(m);
  int32_t* excl = ws.take<int32_t>(m);
  int32_t* lookup = ws.take<int32_t>(m + 8);
  const int64_t scan_bytes = radix::temp_bytes(m);
  void* temp = ws.take<char>(scan_bytes);
  const unsigned blocks = static_cast<unsigned>(ceil_div(m, 256));
  hipLaunchKernelGGL(mask_to_int_kernel, dim3(blocks), dim3(256), 0, stream, mask, m, flags);
  HI3D_HIP_CHECK(radix::scan(temp, scan_bytes, flags, excl, m, false, stream));
  hipLaunchKernelGGL(child_index_kernel, dim3(blocks), dim3(256), 0, stream, mask, excl, m, lookup, parent, slot,
                     n_children);
  static const ChildTables tables = make_child_tables();
  hipLaunchKernelGGL(child_table_kernel, dim3(static_cast<unsigned>(ceil_div(m * 27, 256))), dim3(256), 0, stream,
                     parent_table, lookup, parent, slot, n_children, m, tables, table);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

}  // extern "C"
