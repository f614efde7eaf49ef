// Gather convolution with at most 16 output channels (octree occupancy heads, output
// layers):
//
//   out[o] = act(bias + sum_k in[table[o, k]] . W[:, k, :]^T)  (+ residual[o] after act)
//
// The tile kernels of conv.hip compute 64..256 output channels per tile; with 8 output
// channels most of their MFMA work and all of their weight staging would be padding.
// Here one wave owns 64 output rows (half a plan tile; the plan groups rows by their
// neighbour-presence mask, so the rows of a wave mostly share one mask) as four 16-row
// groups and multiplies with 16x16 MFMAs: the weights are the first operand (output
// channels as the 16 rows, zeros past cout), the gathered input rows the second, so
// lane l's four accumulators of group g are output channels 4*(l/16)..+3 of row slot
// 16*g + l%16. A K step is 64 bytes of every row: lane l reads the 16 bytes at byte
// 16*(l/16) + 64*step of its row for both operands (the contraction only needs both
// operands to split K the same way). Offsets that none of the wave's 64 rows has are
// skipped (a wave-uniform mask); absent entries of a present offset read a 16-byte
// zero vector. Loads go straight to registers, two stages deep; the wave's gather
// indices sit in LDS ([offset][64 rows], 16 consecutive words per read). 16-bit rows of
// a multiple of 128 bytes take conv_narrow_lds_kernel below instead (16-row waves,
// gathers staged through LDS).
//
// Replaces the occupancy head's dense gathered GEMM (SparseClsHead, Conv3d(C, 8):
// src/hi3d_mac/mlx_backend/vae.py:270-271,166-192; src/sparc3d/models/autoencoders/
// blocks.py:181-197).

#include "common.h"
#include "conv_tile.h"

namespace hi3d {
namespace {

constexpr int kNarrowWaves = 4;
constexpr int kNarrowRows = 64;        // output rows per wave
constexpr int kNarrowMaxKvol = 32;
constexpr int kNarrowMaxCout = 16;

__device__ __attribute__((aligned(16))) const uint32_t g_narrow_zero[4] = {0u, 0u, 0u, 0u};

// One 64-byte K step of a 16x16 block: 16 bytes per lane per operand.
template <typename T>
struct Mfma16;

template <>
struct Mfma16<_Float16> {
  __device__ __forceinline__ static void run(u32x4 a, u32x4 b, f32x4& c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

template <>
struct Mfma16<__bf16> {
  __device__ __forceinline__ static void run(u32x4 a, u32x4 b, f32x4& c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                0);
  }
};

// fp32: the 16 bytes are 4 consecutive K values, one 16x16x4 MFMA each.
template <>
struct Mfma16<float> {
  __device__ __forceinline__ static void run(u32x4 a, u32x4 b, f32x4& c) {
    const f32x4 af = __builtin_bit_cast(f32x4, a), bf = __builtin_bit_cast(f32x4, b);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[0], bf[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[1], bf[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[2], bf[2], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[3], bf[3], c, 0, 0, 0);
  }
};

// 16-byte load through a global-address-space pointer (the opaque select of a gathered
// row and the zero vector would otherwise become a flat access, which also counts in
// the LDS counter and makes every wait a full drain).
__device__ __forceinline__ u32x4 gload16(const char* p) {
  return *(const __attribute__((address_space(1))) u32x4*)(p);
}

struct NarrowArgs {
  const char* in;
  const char* w;
  const void* bias;
  const void* residual;
  const int32_t* rows;
  const int32_t* gidx;
  void* out;
  int64_t n_in;
  int64_t n_out;
  int64_t ntiles;
  int32_t cin;
  int32_t cout;
  int32_t kvol;
  int32_t act;
};

template <typename T>
__device__ __forceinline__ float narrow_f32(T v) {
  return static_cast<float>(v);
}

// A stage is CH K steps (64 bytes each) of one present offset: 4 gathered 16-byte
// loads per step (one per 16-row group) and one weight load. Two stages are in flight:
// the loads of stage s + 1 are issued before stage s is multiplied.
template <typename T, int CH>
__global__ __launch_bounds__(kNarrowWaves * 64) void conv_narrow_kernel(NarrowArgs a) {
  __shared__ int32_t entries[kNarrowWaves][kNarrowRows * kNarrowMaxKvol];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  // consecutive wave tiles on one XCD, so that neighbouring rows share its L2
  const int64_t wt = xcd_remap(blockIdx.x, static_cast<int64_t>(gridDim.x)) * kNarrowWaves + wave;
  if (wt >= 2 * a.ntiles) return;  // wave-uniform
  const int64_t slot0 = wt * kNarrowRows;  // first row slot of this wave in the plan
  const int64_t tile = wt >> 1;
  const int half = static_cast<int>(wt & 1);
  const int kvol = a.kvol;
  const uint64_t n_in = static_cast<uint64_t>(a.n_in);
  int32_t* ent = entries[wave];

  // the wave's gather indices into LDS ([offset][64 rows]) and the offsets any of its
  // rows has
  uint32_t present = 0;
  const int32_t* gsrc = a.gidx + tile * kvol * kTileRows + half * kNarrowRows + lane;
  for (int k = 0; k < kvol; ++k) {
    const int32_t e = gsrc[k * kTileRows];
    ent[k * kNarrowRows + lane] = e;
    const bool ok = static_cast<uint64_t>(static_cast<uint32_t>(e)) < n_in;
    present |= __builtin_amdgcn_ballot_w64(ok) != 0 ? (1u << k) : 0u;
  }
  present = __builtin_amdgcn_readfirstlane(present);
  wait_lgkm0();  // the wave reads entries other lanes wrote; only this wave uses its region
  __builtin_amdgcn_wave_barrier();

  const int r = lane & 15, q = lane >> 4;
  const int rb = a.cin * static_cast<int>(sizeof(T));
  const int nch = rb / (64 * CH);
  const char* const zero = reinterpret_cast<const char*>(g_narrow_zero);
  const bool wrow = r < a.cout;
  f32x4 acc[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};

  // stage loads; absent rows (and weight rows past cout) read the zero vector
  auto load = [&](u32x4(&wv)[CH], u32x4(&xv)[CH][4], int k, int c) {
    const int byte0 = c * CH * 64;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int32_t e = ent[k * kNarrowRows + 16 * g + r];
      const bool ok = static_cast<uint64_t>(static_cast<uint32_t>(e)) < n_in;
      uint64_t pin = reinterpret_cast<uint64_t>(a.in) +
                     static_cast<uint64_t>(static_cast<int64_t>(e) * rb + 16 * q + byte0);
      asm volatile("" : "+v"(pin));
      const char* src = ok ? reinterpret_cast<const char*>(pin) : zero;
      const int step = ok ? 64 : 0;
#pragma unroll
      for (int cc = 0; cc < CH; ++cc) xv[cc][g] = gload16(src + cc * step);
    }
    uint64_t wpin = reinterpret_cast<uint64_t>(a.w) +
                    static_cast<uint64_t>((static_cast<int64_t>(r) * kvol + k) * rb + 16 * q + byte0);
    asm volatile("" : "+v"(wpin));
    const char* wsrc = wrow ? reinterpret_cast<const char*>(wpin) : zero;
    const int wstep = wrow ? 64 : 0;
#pragma unroll
    for (int cc = 0; cc < CH; ++cc) wv[cc] = gload16(wsrc + cc * wstep);
  };
  auto compute = [&](const u32x4(&wv)[CH], const u32x4(&xv)[CH][4]) {
#pragma unroll
    for (int cc = 0; cc < CH; ++cc) {
#pragma unroll
      for (int g = 0; g < 4; ++g) Mfma16<T>::run(wv[cc], xv[cc][g], acc[g]);
    }
  };

  const int S = __builtin_popcount(present) * nch;
  if (S > 0) {
    // load cursor; past the last stage it stays there (the extra loads are discarded)
    int kl = __builtin_ctz(present), cl = 0;
    uint32_t rest = present & (present - 1u);
    auto advance = [&]() {
      if (++cl == nch) {
        if (rest) {
          cl = 0;
          kl = __builtin_ctz(rest);
          rest &= rest - 1u;
        } else {
          cl = nch - 1;
        }
      }
    };
    u32x4 wA[CH], xA[CH][4], wB[CH], xB[CH][4];
    load(wA, xA, kl, cl);
    advance();
    // two stages per trip with no exit in between, so the only loads in flight at the
    // top of a trip are those of the stage in A (a mid-trip exit would merge a path
    // with B's loads still in flight into the back edge and make every wait a drain)
    int s = 0;
    for (; s + 2 <= S; s += 2) {
      load(wB, xB, kl, cl);
      advance();
      compute(wA, xA);
      load(wA, xA, kl, cl);
      advance();
      compute(wB, xB);
    }
    if (s < S) compute(wA, xA);  // odd stage count: the last stage is in A
  }

  // epilogue: lane holds channels 4q..4q+3 of row slot 16g + r
  const T* bias = static_cast<const T*>(a.bias);
  const T* res = static_cast<const T*>(a.residual);
  T* out = static_cast<T*>(a.out);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int32_t o = a.rows[slot0 + 16 * g + r];
    if (o < 0 || o >= a.n_out) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 4 * q + i;
      if (j >= a.cout) continue;
      float v = acc[g][i];
      if (bias) v += narrow_f32(bias[j]);
      if (a.act == HI3D_ACT_SILU) v = silu_f32(v);
      T t = static_cast<T>(v);
      const int64_t at = static_cast<int64_t>(o) * a.cout + j;
      if (res) t = static_cast<T>(narrow_f32(t) + narrow_f32(res[at]));
      out[at] = t;
    }
  }
}

// The same convolution for 16-bit rows of a multiple of 128 bytes, with the gathers
// staged through LDS: a wave-wide direct-to-LDS load then covers 8 rows x 128 bytes (8
// full lines) instead of 16 rows x 64 bytes, half the addresser work per byte. Each
// wave (one per workgroup) owns its LDS (gather indices, a 3-slot ring of stages) and
// synchronises with no other wave. A stage is one 128-byte K chunk of one present
// offset: the wave's ROWS gathered rows and the 16 weight rows (zeros past cout),
// ROWS / 8 + WL loads (WL = 1 when cout <= 8: weight rows 8..15 are zeroed once), so
// the vmcnt waits are constants. Rows use the XOR swizzle of the
// tile kernels (chunk c of row r at c ^ ((r >> 1) & 7)), so the 16-row fragment reads
// are free of bank conflicts.
// output rows per wave: more waves per CU outweigh the weight rows each stage reloads
// (occupancy head: 64 rows 0.465 ms, 32 rows 0.423 ms, 16 rows 0.408 ms)
constexpr int kNarrowLdsRows = 16;

__device__ __attribute__((aligned(16))) const uint32_t g_narrow_zero_row[32] = {};

template <typename T, int ROWS, int WL>
__global__ __launch_bounds__(64) void conv_narrow_lds_kernel(NarrowArgs a) {
  constexpr int STAGE = (ROWS + 16) * 128, PARTS = kTileRows / ROWS, G = ROWS / 16;
  constexpr int OPL = 1024 / (ROWS * 4);  // offsets per 16-byte-per-lane index load
  __shared__ __attribute__((aligned(16))) char smem[3 * STAGE + kNarrowMaxKvol * ROWS * 4];
  char* const ring = smem;
  int32_t* const ent = reinterpret_cast<int32_t*>(smem + 3 * STAGE);
  const int lane = threadIdx.x;
  const int64_t wt = xcd_remap(blockIdx.x, static_cast<int64_t>(gridDim.x));
  if (wt >= PARTS * a.ntiles) return;  // wave-uniform
  const int64_t slot0 = wt * ROWS;
  const int64_t tile = wt / PARTS;
  const int half = static_cast<int>(wt % PARTS);
  const int kvol = a.kvol;
  const uint64_t n_in = static_cast<uint64_t>(a.n_in);
  const int rb = a.cin * static_cast<int>(sizeof(T));
  const int nch = rb >> 7;
  if constexpr (WL == 1) {
    // at most 8 outputs: weight rows 8..15 of every ring slot stay zero, and a stage
    // loads rows 0..7 only
#pragma unroll
    for (int sl = 0; sl < 3; ++sl)
      *reinterpret_cast<u32x4*>(smem + sl * STAGE + ROWS * 128 + 1024 + lane * 16) = u32x4{0u, 0u, 0u, 0u};
  }

  // gather indices [offset][ROWS rows]: OPL offsets per 16-byte-per-lane load
  {
    const int groups = (kvol + OPL - 1) / OPL;
    for (int i = 0; i < groups; ++i) {
      int k = OPL * i + lane / (ROWS / 4);
      if (k >= kvol) k = kvol - 1;
      lds_dma16(a.gidx + (tile * kvol + k) * kTileRows + half * ROWS + (lane % (ROWS / 4)) * 4,
                smem + 3 * STAGE + i * 1024);
    }
    wait_vmcnt<0>();
  }
  uint32_t present = 0;
  for (int k = 0; k < kvol; ++k) {
    const bool ok =
        lane < ROWS && static_cast<uint64_t>(static_cast<uint32_t>(ent[k * ROWS + (lane % ROWS)])) < n_in;
    present |= __builtin_amdgcn_ballot_w64(ok) != 0 ? (1u << k) : 0u;
  }
  present = __builtin_amdgcn_readfirstlane(present);

  // load j of a stage covers rows 8 j + lane / 8 at physical chunk lane % 8
  const int lr = lane >> 3, pc = lane & 7;
  const char* const zrow = reinterpret_cast<const char*>(g_narrow_zero_row);
  auto issue = [&](int slot, int k, int c) {
    char* st = ring + slot * STAGE;
#pragma unroll
    for (int j = 0; j < ROWS / 8; ++j) {
      const int row = 8 * j + lr;
      const int lc = pc ^ ((row >> 1) & 7);
      const int32_t e = ent[k * ROWS + row];
      const bool ok = static_cast<uint64_t>(static_cast<uint32_t>(e)) < n_in;
      uint64_t pin = reinterpret_cast<uint64_t>(a.in) + static_cast<uint64_t>(static_cast<int64_t>(e) * rb + c * 128 + lc * 16);
      asm volatile("" : "+v"(pin));
      lds_dma16(ok ? reinterpret_cast<const char*>(pin) : zrow + lc * 16, st + j * 1024);
    }
#pragma unroll
    for (int j = 0; j < WL; ++j) {
      const int o = 8 * j + lr;
      const int lc = pc ^ ((o >> 1) & 7);
      uint64_t wpin = reinterpret_cast<uint64_t>(a.w) +
                      static_cast<uint64_t>((static_cast<int64_t>(o) * kvol + k) * rb + c * 128 + lc * 16);
      asm volatile("" : "+v"(wpin));
      lds_dma16(o < a.cout ? reinterpret_cast<const char*>(wpin) : zrow + lc * 16, st + ROWS * 128 + j * 1024);
    }
  };
  f32x4 acc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int fr = lane & 15, fq = lane >> 4;
  auto compute = [&](int slot) {
    const char* st = ring + slot * STAGE;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int lc = 4 * kk + fq;
      const u32x4 w = *reinterpret_cast<const u32x4*>(st + ROWS * 128 + fr * 128 + ((lc ^ ((fr >> 1) & 7)) << 4));
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int row = 16 * g + fr;
        const u32x4 x = *reinterpret_cast<const u32x4*>(st + row * 128 + ((lc ^ ((row >> 1) & 7)) << 4));
        Mfma16<T>::run(w, x, acc[g]);
      }
    }
  };

  const int S = __builtin_popcount(present) * nch;
  if (S > 0) {
    // issue cursor over (present offset, K chunk)
    int kl = __builtin_ctz(present), cl = 0;
    uint32_t rest = present & (present - 1u);
    auto advance = [&]() {
      if (++cl == nch) {
        cl = 0;
        if (rest) {
          kl = __builtin_ctz(rest);
          rest &= rest - 1u;
        }
      }
    };
    issue(0, kl, cl);
    advance();
    if (S > 1) {
      issue(1, kl, cl);
      advance();
    }
    int slot = 0;
    for (int s = 0; s + 1 < S; ++s) {
      wait_vmcnt<ROWS / 8 + WL>();  // stage s is in LDS; stage s + 1 may still be in flight
      compute(slot);
      if (s + 2 < S) {
        issue(slot == 0 ? 2 : slot - 1, kl, cl);  // the slot of stage s - 1, consumed
        advance();
      }
      slot = slot == 2 ? 0 : slot + 1;
    }
    wait_vmcnt<0>();
    compute(slot);
  }

  // epilogue: lane holds channels 4 fq .. + 3 of row slot 16 g + fr
  const T* bias = static_cast<const T*>(a.bias);
  const T* res = static_cast<const T*>(a.residual);
  T* out = static_cast<T*>(a.out);
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int32_t o = a.rows[slot0 + 16 * g + fr];
    if (o < 0 || o >= a.n_out) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 4 * fq + i;
      if (j >= a.cout) continue;
      float v = acc[g][i];
      if (bias) v += narrow_f32(bias[j]);
      if (a.act == HI3D_ACT_SILU) v = silu_f32(v);
      T t = static_cast<T>(v);
      const int64_t at = static_cast<int64_t>(o) * a.cout + j;
      if (res) t = static_cast<T>(narrow_f32(t) + narrow_f32(res[at]));
      out[at] = t;
    }
  }
}

template <typename T>
int launch_narrow(const NarrowArgs& a, hipStream_t stream) {
  const int64_t blocks = ceil_div(2 * a.ntiles, kNarrowWaves);
  HI3D_REQUIRE(blocks < (int64_t(1) << 31), "too many tiles");
  const int steps = a.cin * static_cast<int>(sizeof(T)) / 64;
  if constexpr (sizeof(T) == 2) {
    if (steps % 2 == 0) {  // 128-byte rows: one wave per workgroup, gathers staged in LDS
      const int64_t waves = (kTileRows / kNarrowLdsRows) * a.ntiles;
      HI3D_REQUIRE(waves < (int64_t(1) << 31), "too many tiles");
      if (a.cout <= 8)
        hipLaunchKernelGGL((conv_narrow_lds_kernel<T, kNarrowLdsRows, 1>), dim3(static_cast<unsigned>(waves)), dim3(64),
                           0, stream, a);
      else
        hipLaunchKernelGGL((conv_narrow_lds_kernel<T, kNarrowLdsRows, 2>), dim3(static_cast<unsigned>(waves)), dim3(64),
                           0, stream, a);
      HI3D_LAUNCH_CHECK();
      return HI3D_OK;
    }
  }
  const dim3 grid(static_cast<unsigned>(blocks)), block(kNarrowWaves * 64);
  if (steps % 2 == 0) {
    hipLaunchKernelGGL((conv_narrow_kernel<T, 2>), grid, block, 0, stream, a);
  } else {
    hipLaunchKernelGGL((conv_narrow_kernel<T, 1>), grid, block, 0, stream, a);
  }
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

}  // namespace
}  // namespace hi3d

using namespace hi3d;

extern "C" int hi3d_gather_conv_narrow(const void* in, int64_t n_in, int32_t cin, const void* weight,
                                       const void* bias, int32_t cout, int32_t kvol, const int32_t* rows,
                                       const int32_t* gidx, const uint32_t* tile_mask, int64_t n_out,
                                       const void* residual, int32_t act, int32_t dtype, void* out, void* stream) {
  (void)tile_mask;  // each wave derives the mask of its own 64 rows from gidx
  HI3D_REQUIRE(dtype == HI3D_F16 || dtype == HI3D_BF16 || dtype == HI3D_F32, "narrow conv takes F16, BF16 or F32");
  const int es = dtype == HI3D_F32 ? 4 : 2;
  HI3D_REQUIRE(cout >= 1 && cout <= kNarrowMaxCout, "narrow conv takes 1..16 output channels, got %d", cout);
  HI3D_REQUIRE(kvol >= 1 && kvol <= kNarrowMaxKvol, "narrow conv takes 1..32 kernel offsets, got %d", kvol);
  HI3D_REQUIRE(cin > 0 && (static_cast<int64_t>(cin) * es) % 64 == 0,
               "narrow conv needs input rows of a multiple of 64 bytes (cin %d)", cin);
  HI3D_REQUIRE(n_in >= 0 && n_out >= 0 && n_in < (int64_t(1) << 31) - 1 && n_out < (int64_t(1) << 31) - 1,
               "bad sizes");
  HI3D_REQUIRE(act == HI3D_ACT_NONE || act == HI3D_ACT_SILU, "unknown activation %d", act);
  if (n_out == 0) return HI3D_OK;
  HI3D_REQUIRE(in && weight && rows && gidx && out, "null pointer argument");
  HI3D_REQUIRE(reinterpret_cast<uintptr_t>(in) % 16 == 0 && reinterpret_cast<uintptr_t>(weight) % 16 == 0,
               "input and weight must be 16-byte aligned");
  NarrowArgs a{static_cast<const char*>(in), static_cast<const char*>(weight), bias, residual, rows, gidx, out,
               n_in, n_out, ceil_div(n_out, kTileRows), cin, cout, kvol, act};
  hipStream_t s = as_stream(stream);
  switch (dtype) {
    case HI3D_F16: return launch_narrow<_Float16>(a, s);
    case HI3D_BF16: return launch_narrow<__bf16>(a, s);
    default: return launch_narrow<float>(a, s);
  }
}
