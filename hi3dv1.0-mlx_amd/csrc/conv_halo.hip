// Gather convolution over halo plans (3x3x3 submanifold maps, fp16 / bf16, Cout a
// multiple of 128, 256..512-byte input rows).
//
// A tile is 256 output rows in Morton order. The input rows that any of its 27 offsets
// touch (its halo, at most 767 rows) are gathered into LDS once per 64-byte K step, and
// every offset then reads its rows from there through the plan's per-(row, offset) halo
// positions: each input row leaves HBM once per tile and K step instead of once per
// (output row, offset), and the gathers become L2/LDS traffic.
//  * Workgroup: 8 waves; wave (wm, th) owns rows 64 wm .. +63 and all 128 channels as
//    4 x 2 blocks of 32x32x16 MFMAs (weights as the first operand) over the even (th 0)
//    or odd (th 1) offsets. Halving the offsets per wave rather than the channels halves
//    the reads of randomly placed halo rows (LDS bank conflicts) per MFMA; the two
//    partial sums of a row meet once per tile through LDS (fp32 addition commutes, so
//    the result does not depend on which wave adds).
//  * LDS: two halo slots of 768 rows x 64 bytes (K steps kb and kb + 1) and a 3-deep
//    ring of weight stages (two offsets x 128 rows x 64 bytes). Rows use the 64-byte
//    swizzled layout (chunk c of row r at c ^ ((r >> 1 ^ r >> 3) & 3)); halo row 767 is
//    always absent and reads as zeros, standing in for absent (row, offset) pairs.
//  * Stages: (K step kb, offset pair). One barrier per stage; after it the stage's
//    loads two stages ahead are issued (two weight loads per wave) and, during stages
//    1..6 of a K step, one of the wave's six halo loads of the next K step. Every wave
//    issues the same loads, so the vmcnt waits are exact: at stage s the loads younger
//    than stage s's weights are stage s + 1's two and the halo load of stage s - 1.
//  * Epilogue: each wave hands the partner (same rows, other offsets) the channel half it
//    does not finish and adds the partner's half of its own; then bias + activation in
//    fp32, round to T, and each wave stages its 64 x 64 block in LDS and writes 16-byte
//    row chunks to the tile's output rows, adding the residual.
#include <type_traits>

#include "common.h"
#include "conv_tile.h"

namespace hi3d {
namespace {

constexpr int kHRows = 256;
constexpr int kHMax = 768;
constexpr int kHKvol = 27;
constexpr int kHThreads = 512;
constexpr int kHSlot = kHMax * 64;
constexpr int kHStageB = 2 * 128 * 64;
constexpr int kHRingB = 3;
constexpr int kHPairs = (kHKvol + 1) / 2;
constexpr int kHMaxRowBytes = 512;

struct HaloArgs {
  const char* in;
  int64_t n_in;
  int32_t cin;
  const char* weight;
  const void* bias;
  int32_t cout;
  const int32_t* rows;
  const int32_t* halo;
  const uint16_t* loff;
  int64_t ntiles;
  int32_t ny;
  const char* residual;
  int32_t act;
  char* out;
};

__device__ __attribute__((aligned(16))) const uint32_t g_halo_zero[kHMaxRowBytes / 4] = {};

__device__ __forceinline__ int hoff(int row, int chunk) {
  return row * 64 + ((chunk ^ ((row >> 2) & 3)) << 4);
}

template <typename T>
__global__ __launch_bounds__(kHThreads, 1) void conv_halo_kernel(HaloArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[2 * kHSlot + kHRingB * kHStageB];
  char* const bring = smem + 2 * kHSlot;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 3, th = wave >> 2;
  const int64_t item = xcd_remap(blockIdx.x, static_cast<int64_t>(gridDim.x));
  const int64_t tile = item / a.ny;
  const int n0 = static_cast<int>(item - tile * a.ny) * 128;
  const int rb = a.cin * static_cast<int>(sizeof(T));
  const int KB = rb >> 6;
  const int S = kHPairs * KB;
  const uint64_t n_in = static_cast<uint64_t>(a.n_in);
  const char* const zero = reinterpret_cast<const char*>(g_halo_zero);

  // halo loads: load j (0..5) of this wave covers halo rows (wave + 8 j) * 16 .. +15; lane
  // l fills row + l / 4 at physical chunk l % 4 (logical chunk (l % 4) ^ swizzle)
  const char* hsrc[6];
#pragma unroll
  for (int j = 0; j < 6; ++j) {
    const int hr = (wave + 8 * j) * 16 + (lane >> 2);
    const int c = (lane & 3) ^ ((hr >> 2) & 3);
    const int32_t g = a.halo[tile * kHMax + hr];
    hsrc[j] = static_cast<uint64_t>(static_cast<uint32_t>(g)) < n_in ? a.in + static_cast<int64_t>(g) * rb + c * 16
                                                                       : zero + c * 16;
  }
  // weight loads: load u (offset u of the pair) covers weight rows 16 wave .. +15
  const int br = wave * 16 + (lane >> 2);
  const int bc = (lane & 3) ^ ((br >> 2) & 3);
  const char* const wsrc = a.weight + static_cast<int64_t>(n0 + br) * kHKvol * rb + bc * 16;
  const char* const wzero = zero + bc * 16;
  // A-fragment LDS offsets of this wave's offsets k = 2 p + th (K-group 0; K-group 1 is
  // offset ^ 32): rows 64 wm + 32 mb + l % 32, packed as mb 0 in bits 0..15, mb 1 in 16..31
  uint32_t aoff[kHPairs];
#pragma unroll
  for (int p = 0; p < kHPairs; ++p) aoff[p] = 0;
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
    const int lr = wm * 64 + mb * 32 + (lane & 31);
    const u32x4* lp = reinterpret_cast<const u32x4*>(a.loff + (tile * kHRows + lr) * 32);
    u32x4 v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = lp[i];
#pragma unroll
    for (int p = 0; p < kHPairs; ++p) {
      // offset k = 2 p + th: halfword th of word p
      const uint32_t word = v[p >> 2][p & 3];
      const uint32_t lid = th ? (word >> 16) : (word & 0xffffu);
      const int h = (lid == 0xffffu || 2 * p + th >= kHKvol) ? kHMax - 1 : static_cast<int>(lid);
      aoff[p] |= static_cast<uint32_t>(hoff(h, lane >> 5)) << (16 * mb);
    }
  }

  auto issue_b = [&](int s) {  // weights of stage s (K step s / 14, offset pair s % 14)
    const int kb = s / kHPairs, pr = s - kb * kHPairs;
    char* dst = bring + (s % kHRingB) * kHStageB + wave * 1024;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int k = 2 * pr + u;
      int off = k * rb + kb * 64;
      asm volatile("" : "+s"(off));  // keeps per-offset source pointers from being precomputed
      lds_dma16(k < kHKvol ? wsrc + off : wzero, dst + u * (kHStageB / 2));
    }
  };
  auto issue_h = [&](int kb, int j) {
    lds_dma16(hsrc[j] + kb * 64, smem + (kb & 1) * kHSlot + (wave + 8 * j) * 1024);
  };

  f32x16 acc[4][2];  // [channel block][row block]
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[nb][mb][v] = 0.0f;

  // prologue: halo K step 0, weights of stages 0 and 1
#pragma unroll
  for (int j = 0; j < 6; ++j) issue_h(0, j);
  issue_b(0);
  if (S > 1) issue_b(1);

  for (int kb = 0; kb < KB; ++kb) {
    const char* hs = smem + (kb & 1) * kHSlot;
    const bool more_kb = kb + 1 < KB;
#pragma unroll
    for (int pr = 0; pr < kHPairs; ++pr) {
      const int s = kb * kHPairs + pr;
      // wait for stage s's weights (and, at pr 0, this K step's halo)
      const bool h_prev = pr >= 2 && pr <= 7 && more_kb;  // a halo load was issued in stage s - 1
      if (s + 1 < S) {
        if (h_prev) wait_vmcnt<3>();
        else wait_vmcnt<2>();
      } else {
        if (h_prev) wait_vmcnt<1>();
        else wait_vmcnt<0>();
      }
      raw_barrier();
      if (s + 2 < S) issue_b(s + 2);
      if (pr >= 1 && pr <= 6 && more_kb) issue_h(kb + 1, pr - 1);
      const char* bs = bring + (s % kHRingB) * kHStageB + th * (kHStageB / 2);
      // this wave's offset k = 2 pr + th (the last pair has no odd offset); K-groups g 0, 1
      if (2 * pr + th < kHKvol) {
        uint32_t word = aoff[pr];
        asm volatile("" : "+v"(word));  // unpacked per use, not precomputed for all offsets
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          u32x4 fa[2], fb[4];
#pragma unroll
          for (int mb = 0; mb < 2; ++mb)
            fa[mb] = *reinterpret_cast<const u32x4*>(hs + (((word >> (16 * mb)) & 0xffffu) ^ (g << 5)));
#pragma unroll
          for (int nb = 0; nb < 4; ++nb)
            fb[nb] = *reinterpret_cast<const u32x4*>(bs + hoff(nb * 32 + (lane & 31), 2 * g + (lane >> 5)));
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int nb = 0; nb < 4; ++nb)
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) Mfma<T>::run(fb[nb], fa[mb], acc[nb][mb]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  }

  // epilogue: exchange channel halves with the partner wave (same rows, other offsets)
  wait_vmcnt<0>();
  __syncthreads();
  auto exchange = [&](auto tc) {  // tc: this wave's offset parity as a compile-time constant
    constexpr int kTh = decltype(tc)::value;
    constexpr int kGive = kTh ? 0 : 2, kKeep = kTh ? 2 : 0;  // th 0 keeps channel blocks 0, 1
    char* mine = smem + wave * 16384;  // the half the partner finishes
    const char* theirs = smem + (wave ^ 4) * 16384;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 v = {acc[kGive + i][mb][4 * q], acc[kGive + i][mb][4 * q + 1], acc[kGive + i][mb][4 * q + 2],
                           acc[kGive + i][mb][4 * q + 3]};
          *reinterpret_cast<f32x4*>(mine + ((i * 2 + mb) * 4 + q) * 1024 + lane * 16) = v;
        }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(theirs + ((i * 2 + mb) * 4 + q) * 1024 + lane * 16);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[kKeep + i][mb][4 * q + e] += v[e];
        }
    __syncthreads();
  };
  if (th) exchange(std::integral_constant<int, 1>{});
  else exchange(std::integral_constant<int, 0>{});
  const int wn = th;  // channels n0 + 64 wn .. +63 are finished by this wave
  const T* bias = static_cast<const T*>(a.bias);
  char* stg = smem + wave * (64 * 128);  // this wave's 64 rows x 64 channels
  auto finish = [&](auto tc) {
    constexpr int kWn = decltype(tc)::value;
#pragma unroll
    for (int nbl = 0; nbl < 2; ++nbl) {
      const int nb = 2 * kWn + nbl;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int j0 = nbl * 32 + 8 * q + 4 * (lane >> 5);  // channel within the wave's 64
        float b[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) b[e] = bias != nullptr ? static_cast<float>(bias[n0 + kWn * 64 + j0 + e]) : 0.0f;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
          const int row = mb * 32 + (lane & 31);
          T h[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float x = acc[nb][mb][4 * q + e] + b[e];
            if (a.act == HI3D_ACT_SILU) x = silu_f32(x);
            h[e] = static_cast<T>(x);
          }
          uint2 packed;
          __builtin_memcpy(&packed, h, 8);
          *reinterpret_cast<uint2*>(stg + row * 128 + (((j0 >> 3) ^ (row & 7)) << 4) + (j0 & 4) * 2) = packed;
        }
      }
    }
  };
  if (wn) finish(std::integral_constant<int, 1>{});
  else finish(std::integral_constant<int, 0>{});
  wait_lgkm0();
  const int64_t out_row_bytes = static_cast<int64_t>(a.cout) * sizeof(T);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = (lane >> 3) + 8 * i;  // 0..63 within this wave's rows
    const int chunk = lane & 7;
    const int32_t orow = a.rows[tile * kHRows + wm * 64 + row];
    if (orow < 0) continue;
    u32x4 v = *reinterpret_cast<const u32x4*>(stg + row * 128 + ((chunk ^ (row & 7)) << 4));
    const int64_t off =
        static_cast<int64_t>(orow) * out_row_bytes + static_cast<int64_t>(n0 + wn * 64 + chunk * 8) * sizeof(T);
    if (a.residual != nullptr) {
      const u32x4 r = *reinterpret_cast<const u32x4*>(a.residual + off);
      T* pv = reinterpret_cast<T*>(&v);
      const T* pr = reinterpret_cast<const T*>(&r);
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = static_cast<T>(static_cast<float>(pv[e]) + static_cast<float>(pr[e]));
    }
    *reinterpret_cast<u32x4*>(a.out + off) = v;
  }
}

template <typename T>
int launch_halo(const HaloArgs& base, hipStream_t stream) {
  HaloArgs a = base;
  a.ny = a.cout / 128;
  const int64_t blocks = a.ntiles * a.ny;
  if (blocks == 0) return HI3D_OK;
  HI3D_REQUIRE(blocks < (int64_t(1) << 31), "too many tiles");
  hipLaunchKernelGGL((conv_halo_kernel<T>), dim3(static_cast<unsigned>(blocks)), dim3(kHThreads), 0, stream, a);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

}  // namespace
}  // namespace hi3d

using namespace hi3d;

extern "C" {

int hi3d_halo_conv(const void* in_dev, int64_t n_in, int32_t cin, const void* weight_dev, const void* bias_dev,
                   int32_t cout, const int32_t* rows_dev, const int32_t* halo_dev, const uint16_t* loff_dev,
                   int64_t ntiles, const void* residual_dev, int32_t act, int32_t dtype, void* out_dev,
                   void* stream_) {
  hipStream_t stream = as_stream(stream_);
  HI3D_REQUIRE(dtype == HI3D_F16 || dtype == HI3D_BF16, "the halo convolution takes fp16 or bf16");
  HI3D_REQUIRE(cout > 0 && cout % 128 == 0, "Cout must be a multiple of 128 (got %d)", cout);
  const int64_t rb = static_cast<int64_t>(cin) * 2;
  HI3D_REQUIRE(cin > 0 && rb % 64 == 0 && rb >= 4 * 64 && rb <= kHMaxRowBytes,
               "Cin must give 256..512-byte rows in 64-byte steps (got %d)", cin);
  HI3D_REQUIRE(n_in >= 0 && n_in < (int64_t(1) << 31) - 1, "bad n_in");
  HI3D_REQUIRE(act == HI3D_ACT_NONE || act == HI3D_ACT_SILU, "unknown activation %d", act);
  HI3D_REQUIRE(ntiles >= 0, "bad ntiles");
  if (ntiles == 0) return HI3D_OK;
  HI3D_REQUIRE(in_dev && weight_dev && rows_dev && halo_dev && loff_dev && out_dev, "null pointer argument");
  const uintptr_t align = reinterpret_cast<uintptr_t>(in_dev) | reinterpret_cast<uintptr_t>(weight_dev) |
                          reinterpret_cast<uintptr_t>(out_dev) | reinterpret_cast<uintptr_t>(residual_dev) |
                          reinterpret_cast<uintptr_t>(loff_dev);
  HI3D_REQUIRE((align & 15) == 0, "features, weight, output, residual and the plan must be 16-byte aligned");
  HaloArgs a{static_cast<const char*>(in_dev), n_in, cin, static_cast<const char*>(weight_dev), bias_dev, cout,
             rows_dev, halo_dev, loff_dev, ntiles, 1, static_cast<const char*>(residual_dev), act,
             static_cast<char*>(out_dev)};
  return dtype == HI3D_F16 ? launch_halo<_Float16>(a, stream) : launch_halo<__bf16>(a, stream);
}

}  // extern "C"
