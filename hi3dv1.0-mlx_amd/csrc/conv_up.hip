// Transposed 2x2x2 / stride-2 convolution onto the fine set, parent-major:
//
//   z[child(c, s)] = b + W[:, s, :] y[c]   for every coarse row c and present slot s.
//
// Every fine row has exactly one parent, so the gather formulation over the fine rows
// reads each coarse row once per child (about 3.4 times, far apart in the plan's slot
// groups). Here a workgroup walks tiles of 32 consecutive coarse rows: the rows arrive
// by direct-to-LDS loads as one contiguous block, each of the 4 waves multiplies them
// by the weights of two slots, kept in registers for the whole launch, and writes the
// rows of the children that exist. Each coarse row is read once and each fine row
// written once.
//
// Sorted form (kSorted): a plan orders the coarse rows by their children's slot mask
// (``hi3d_stride2_up_plan``, a radix sort of the 8-bit masks), so the 32 rows of a tile
// mostly share one mask, and a wave skips the MFMAs of its slots that no row of the
// tile has (on thin shells 3.4 of a row's 8 slots hold a child, so contiguous tiles have
// every slot somewhere and compute all 8). The tile's rows are then gathered by their
// indices: each wave fetches the indices of the tile R - 1 ahead into its own LDS ring
// slot with its first load of a tile, so they have landed (its own waits cover them)
// by the time the rows are issued. The child table arrives pre-permuted, contiguous per
// tile. Results are those of the contiguous form, bit for bit (each child is computed
// by the same MFMA sequence).
//
// Tiles run through a 6-deep LDS ring, five tiles ahead of the one being computed (4-
// and 7-deep rings measured the same). The epilogue stays in registers: one lane swap
// turns the MFMA's 4-channel pieces into 16-byte chunks (staging the rows in LDS for
// whole-line stores was 10 % slower). A wave issues the same number of loads and stores
// per tile (stores of absent children go to an out-of-range offset of a bounded buffer
// resource and are dropped), so the vmcnt waits are exact constants.
#include <algorithm>

#include "common.h"
#include "conv_tile.h"
#include "radix.h"

namespace hi3d {
namespace {

constexpr int kUpParents = 32;  // coarse rows per tile
constexpr int kUpWaves = 4;     // each holds the weights of two slots
constexpr uint32_t kBufferFlags = 0x00020000u;  // raw 32-bit buffer (gfx9 descriptor word 3)
constexpr int kUpRing = 6;      // tile buffers per workgroup

template <int CIN, int COUT>
struct UpShape {
  static constexpr int RB = CIN * 2;                          // input row bytes
  static constexpr int CPR = RB / 16;                         // 16-byte chunks per input row
  static constexpr int ROWS = kUpParents * RB;                // bytes of a tile's rows
  static constexpr int DOWN = kUpParents * 8 * 4;             // the tile's child table rows
  static constexpr int BUF = ROWS + DOWN;                     // one ring buffer
  static constexpr int NLR = ROWS / (kUpWaves * 1024);        // 16-byte row DMAs per wave
  static constexpr int NL = NLR + 1;                          // + one 4-byte DMA of child rows
  static constexpr int KS = CIN / 16;                         // MFMA K steps
  static constexpr int OB = COUT / 32;                        // 32-channel output blocks
  static constexpr int ROWO = COUT * 2;                       // output row bytes
  static constexpr int NS = 2 * OB * 2;                       // stores per wave and tile
  static_assert(ROWS % (kUpWaves * 1024) == 0 && DOWN == kUpWaves * 256, "tile shape");
  static_assert(CPR == 8 || CPR == 16, "input rows of 128 or 256 bytes");
};

// position of logical 16-byte chunk c of tile row r: 16 consecutive rows read at one
// chunk fall in 16 distinct 4-bank groups
template <int CPR>
__device__ __forceinline__ int up_chunk(int r, int c) {
  if constexpr (CPR == 16)
    return c ^ (r & 15);
  else
    return c ^ ((r >> 1) & 7);
}

__device__ __forceinline__ void up_dma4(const void* src, char* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(lds_wave_base), 4, 0, 0);
}

template <typename T>
__device__ __forceinline__ float up_f32(T v) {
  return static_cast<float>(v);
}

struct UpArgs {
  const char* in;        // [n_c, cin] coarse rows
  const char* weight;    // [cout, 8, cin]
  const void* bias;      // [cout] or null
  const int32_t* down;   // [n_c, 8] child row per slot, >= n_f absent (sorted: [ntiles * 32, 8], permuted)
  const int32_t* order;  // sorted form: [ntiles * 32] coarse row of each tile position
  char* out;             // [n_f, cout]
  int64_t n_c, n_f, ntiles;
  uint32_t out_bytes;
};

template <typename T, int CIN, int COUT, bool kSorted>
__global__ __launch_bounds__(kUpWaves * 64, 2) void conv_up_kernel(UpArgs a) {
  using Sh = UpShape<CIN, COUT>;
  constexpr int R = kUpRing, NL = Sh::NL + (kSorted ? 1 : 0), NS = Sh::NS, KS = Sh::KS, OB = Sh::OB;
  constexpr int ORD = kSorted ? R * kUpWaves * 256 : 0;  // per (ring slot, wave): the tile's 32 row indices (x2)
  static_assert(NS + (R - 2) * (NL + NS) < 64, "vmcnt is a 6-bit counter");
  // one LDS object: with several, the compiler's alias scopes make it wait for every
  // outstanding direct-to-LDS load before each LDS read
  __shared__ __attribute__((aligned(16))) char smem[R * Sh::BUF + ORD + COUT * 4];
  char* const ord_base = smem + R * Sh::BUF;
  float* const bias_lds = reinterpret_cast<float*>(smem + R * Sh::BUF + ORD);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // the weights of slots 2 wave and 2 wave + 1 as first MFMA operands: lane l holds
  // output channel 32 ob + l % 32, input channels 16 k + 8 (l / 32) .. + 7
  u32x4 wf[2][OB][KS];
#pragma unroll
  for (int si = 0; si < 2; ++si)
#pragma unroll
    for (int ob = 0; ob < OB; ++ob)
#pragma unroll
      for (int k = 0; k < KS; ++k) {
        const int co = ob * 32 + (lane & 31), s = 2 * wave + si;
        wf[si][ob][k] = *reinterpret_cast<const u32x4*>(
            a.weight + (static_cast<int64_t>(co) * 8 + s) * Sh::RB + (16 * k + 8 * (lane >> 5)) * 2);
      }
  // the bias in fp32 (LDS keeps it out of the registers the weights fill; the first
  // barrier of the tile loop orders these writes before every read)
  if (threadIdx.x < COUT)
    bias_lds[threadIdx.x] = a.bias != nullptr ? up_f32(static_cast<const T*>(a.bias)[threadIdx.x]) : 0.0f;
  wait_lgkm0();
  const __amdgpu_buffer_rsrc_t out_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(a.out, 0, static_cast<int>(a.out_bytes), static_cast<int>(kBufferFlags));

  const int64_t first = blockIdx.x, step = gridDim.x;
  const int64_t count = first < a.ntiles ? (a.ntiles - 1 - first) / step + 1 : 0;

  // sorted form: this wave's copy of the row indices of local tile i (lanes 32..63
  // repeat lanes 0..31) into ring slot i % R
  auto order_dma = [&](int64_t i) {
    int64_t t = first + i * step;
    if (t >= a.ntiles) t = a.ntiles - 1;
    up_dma4(a.order + t * kUpParents + (lane & 31), ord_base + (static_cast<int>(i % R) * kUpWaves + wave) * 256);
  };
  // loads of the i-th tile of this workgroup (the last tile again past the end; such a
  // buffer is never read) into ring buffer i % R; sorted: first the indices of tile
  // i + R - 1 (read when that tile is issued, after this wave's wait for tile i)
  auto issue = [&](int64_t i) {
    if constexpr (kSorted) order_dma(i + R - 1);
    int64_t t = first + i * step;
    if (t >= a.ntiles) t = a.ntiles - 1;
    const int64_t c0 = t * kUpParents;
    char* buf = smem + static_cast<int>(i % R) * Sh::BUF;
    const int32_t* ord =
        reinterpret_cast<const int32_t*>(ord_base + (static_cast<int>(i % R) * kUpWaves + wave) * 256);
#pragma unroll
    for (int j = 0; j < Sh::NLR; ++j) {
      const int u = (j * kUpWaves + wave) * 64 + lane;  // 16-byte unit of the tile
      const int r = u / Sh::CPR, cp = u % Sh::CPR;
      int64_t row;
      if constexpr (kSorted) {
        row = ord[r];  // the plan pads with a valid row
      } else {
        row = c0 + r;
        if (row >= a.n_c) row = a.n_c - 1;
      }
      lds_dma16(a.in + row * Sh::RB + up_chunk<Sh::CPR>(r, cp) * 16, buf + (j * kUpWaves + wave) * 1024);
    }
    int64_t prow = c0 + wave * 8 + (lane >> 3);
    if (!kSorted && prow >= a.n_c) prow = a.n_c - 1;  // the sorted table is padded to whole tiles
    up_dma4(a.down + prow * 8 + (lane & 7), buf + Sh::ROWS + wave * 256);
  };

  wait_vmcnt<0>();  // the weights, before any tile load is in flight
  if (count > 0) {
    if constexpr (kSorted) {
#pragma unroll
      for (int i = 0; i < R - 1; ++i) order_dma(i);
      wait_vmcnt<0>();
    }
#pragma unroll
    for (int i = 0; i < R - 1; ++i) issue(i);
  }
  for (int64_t it = 0; it < count; ++it) {
    // loads issued after tile it's: (R - 2) tiles' loads plus, once the pipeline is
    // full, R - 1 tiles' stores
    if (it < R - 1)
      wait_vmcnt<(R - 2) * NL>();
    else
      wait_vmcnt<NS + (R - 2) * (NL + NS)>();
    raw_barrier();  // every wave's part of tile it is in LDS; buffer (it - 1) % R is free
    issue(it + R - 1);

    const char* buf = smem + static_cast<int>(it % R) * Sh::BUF;
    const int64_t c0 = (first + it * step) * kUpParents;
    const int32_t* dn = reinterpret_cast<const int32_t*>(buf + Sh::ROWS);
    const int p = lane & 31, h = lane >> 5;
    // the children of this lane's tile row in the wave's two slots; a slot that no row
    // of the tile has skips its MFMAs (its stores go out of range like every absent one)
    int32_t child[2];
    bool ok[2], has[2];
#pragma unroll
    for (int si = 0; si < 2; ++si) {
      child[si] = dn[p * 8 + 2 * wave + si];
      ok[si] = c0 + p < a.n_c &&
               static_cast<uint64_t>(static_cast<uint32_t>(child[si])) < static_cast<uint64_t>(a.n_f);
      has[si] = __ballot(ok[si]) != 0;
    }
    f32x16 acc[2][OB];
#pragma unroll
    for (int si = 0; si < 2; ++si)
#pragma unroll
      for (int ob = 0; ob < OB; ++ob)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[si][ob][v] = 0.0f;
#pragma unroll
    for (int k = 0; k < KS; ++k) {
      const int r = lane & 31, c = 2 * k + (lane >> 5);
      const u32x4 b = *reinterpret_cast<const u32x4*>(buf + r * Sh::RB + up_chunk<Sh::CPR>(r, c) * 16);
#pragma unroll
      for (int si = 0; si < 2; ++si)
        if (has[si]) {
#pragma unroll
          for (int ob = 0; ob < OB; ++ob) Mfma<T>::run(wf[si][ob][k], b, acc[si][ob]);
        }
    }

    // epilogue in registers: lanes l and l + 32 hold channels 8 q + 0..3 and 8 q + 4..7
    // of parent l % 32; one lane swap per pair (q, q + 1) gives lane l channels
    // 16 m + 0..7 and lane l + 32 channels 16 m + 8..15, a 16-byte chunk each
    // (v_permlane32_swap exchanges lanes 32..63 of its first operand with lanes 0..31
    // of its second)
#pragma unroll
    for (int si = 0; si < 2; ++si) {
#pragma unroll
      for (int ob = 0; ob < OB; ++ob) {
        uint32_t pk[4][2];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 bv = *reinterpret_cast<const f32x4*>(bias_lds + ob * 32 + 8 * q + 4 * h);
          T hv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) hv[e] = static_cast<T>(acc[si][ob][4 * q + e] + bv[e]);
          __builtin_memcpy(pk[q], hv, 8);
        }
#pragma unroll
        for (int m = 0; m < 2; ++m) {
#pragma unroll
          for (int d = 0; d < 2; ++d) {
            const auto sw = __builtin_amdgcn_permlane32_swap(pk[2 * m][d], pk[2 * m + 1][d], false, false);
            pk[2 * m][d] = sw[0];
            pk[2 * m + 1][d] = sw[1];
          }
          const u32x4 v = {pk[2 * m][0], pk[2 * m][1], pk[2 * m + 1][0], pk[2 * m + 1][1]};
          const int chunk = 4 * ob + 2 * m + h;
          const uint32_t off = ok[si]
                                   ? static_cast<uint32_t>(child[si]) * static_cast<uint32_t>(Sh::ROWO) + chunk * 16
                                   : a.out_bytes;
          __builtin_amdgcn_raw_buffer_store_b128(v, out_rsrc, static_cast<int>(off), 0, 0);
        }
      }
    }
  }
  wait_vmcnt<0>();
}

template <typename T, int CIN, int COUT, bool kSorted>
int launch_up(const UpArgs& a, hipStream_t stream) {
  // persistent workgroups: as many as fit on the chip at once (each walks its tiles)
  static int per_cu[2][64] = {};
  int dev = 0;
  HI3D_HIP_CHECK(hipGetDevice(&dev));
  if (dev >= 0 && dev < 64 && per_cu[kSorted][dev] == 0)
    HI3D_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu[kSorted][dev],
                                                                conv_up_kernel<T, CIN, COUT, kSorted>,
                                                                kUpWaves * 64, 0));
  const int fit = dev >= 0 && dev < 64 && per_cu[kSorted][dev] > 0 ? per_cu[kSorted][dev] : 1;
  const int64_t blocks = std::min<int64_t>(a.ntiles, static_cast<int64_t>(compute_units()) * fit);
  hipLaunchKernelGGL((conv_up_kernel<T, CIN, COUT, kSorted>), dim3(static_cast<unsigned>(blocks)),
                     dim3(kUpWaves * 64), 0, stream, a);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

template <typename T, bool kSorted>
int dispatch_up(const UpArgs& a, int cin, hipStream_t stream) {
  if (cin == 128) return launch_up<T, 128, 64, kSorted>(a, stream);
  return launch_up<T, 64, 64, kSorted>(a, stream);
}

// Plan of the sorted form: key = (row >> window_log2) << 8 | slot mask of the row's
// children, so a stable sort groups rows of one mask inside each window of rows.
__global__ void up_keys_kernel(const int32_t* __restrict__ down, int64_t n_c, int64_t n_f, int window_log2,
                               uint32_t* __restrict__ keys, int32_t* __restrict__ rows) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c >= n_c) return;
  uint32_t mask = 0;
#pragma unroll
  for (int s = 0; s < 8; ++s)
    mask |= (static_cast<uint64_t>(static_cast<uint32_t>(down[c * 8 + s])) < static_cast<uint64_t>(n_f) ? 1u : 0u)
            << s;
  keys[c] = (static_cast<uint32_t>(c >> window_log2) << 8) | mask;
  rows[c] = static_cast<int32_t>(c);
}

// order[i] = the i-th sorted row (padding: row n_c - 1, a valid address) and its child
// table row (padding: every slot absent).
__global__ void up_order_kernel(const int32_t* __restrict__ sorted, const int32_t* __restrict__ down, int64_t n_c,
                                int64_t n_f, int64_t npad, int32_t* __restrict__ order,
                                int32_t* __restrict__ down_sorted) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= npad) return;
  const int32_t p = i < n_c ? sorted[i] : -1;
  order[i] = p >= 0 ? p : static_cast<int32_t>(n_c - 1);
#pragma unroll
  for (int s = 0; s < 8; ++s) down_sorted[i * 8 + s] = p >= 0 ? down[static_cast<int64_t>(p) * 8 + s] : static_cast<int32_t>(n_f);
}

int up_check(int32_t cin, int32_t cout, int32_t dtype, int64_t n_c, int64_t n_f) {
  HI3D_REQUIRE(hi3d_stride2_up_supported(cin, cout, dtype),
               "parent-major up convolution takes F16 / BF16, cin 64 or 128, cout 64; got (%d, %d), dtype %d", cin,
               cout, dtype);
  HI3D_REQUIRE(n_c >= 0 && n_f >= 0 && n_c < (int64_t(1) << 31) - 1, "bad sizes");
  HI3D_REQUIRE(n_f * cout * 2 < (int64_t(1) << 31), "output of %lld rows exceeds 2 GiB", static_cast<long long>(n_f));
  return HI3D_OK;
}

}  // namespace
}  // namespace hi3d

using namespace hi3d;

extern "C" {

int hi3d_stride2_up_supported(int32_t cin, int32_t cout, int32_t dtype) {
  return (dtype == HI3D_F16 || dtype == HI3D_BF16) && (cin == 128 || cin == 64) && cout == 64;
}

int hi3d_stride2_up_tile_rows(void) { return kUpParents; }

int hi3d_stride2_up_conv(const void* in, int64_t n_c, int32_t cin, const void* weight, const void* bias, int32_t cout,
                         const int32_t* down, int64_t n_f, int32_t dtype, void* out, void* stream) {
  int rc = up_check(cin, cout, dtype, n_c, n_f);
  if (rc != HI3D_OK) return rc;
  if (n_c == 0 || n_f == 0) return HI3D_OK;
  HI3D_REQUIRE(in && weight && down && out, "null pointer argument");
  HI3D_REQUIRE(((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(weight) |
                 reinterpret_cast<uintptr_t>(out)) & 15) == 0,
               "input, weight and output must be 16-byte aligned");
  UpArgs a{static_cast<const char*>(in), static_cast<const char*>(weight), bias, down, nullptr,
           static_cast<char*>(out), n_c, n_f, ceil_div(n_c, kUpParents), static_cast<uint32_t>(n_f * cout * 2)};
  hipStream_t s = as_stream(stream);
  if (dtype == HI3D_BF16) return dispatch_up<__bf16, false>(a, cin, s);
  return dispatch_up<_Float16, false>(a, cin, s);
}

int hi3d_stride2_up_plan_workspace(int64_t n_c, int64_t* bytes) {
  HI3D_REQUIRE(bytes != nullptr, "bytes_host is NULL");
  HI3D_REQUIRE(n_c >= 0 && n_c < (int64_t(1) << 31) - 1, "bad coarse row count");
  const int64_t m = std::max<int64_t>(n_c, 1);
  *bytes = 4 * align_up(m * 4, 256) + radix::temp_bytes(m);
  return HI3D_OK;
}

int hi3d_stride2_up_plan(const int32_t* down, int64_t n_c, int64_t n_f, int32_t window_log2, void* workspace,
                         int64_t workspace_bytes, int32_t* order, int32_t* down_sorted, void* stream_) {
  hipStream_t stream = as_stream(stream_);
  int64_t need = 0;
  int rc = hi3d_stride2_up_plan_workspace(n_c, &need);
  if (rc != HI3D_OK) return rc;
  HI3D_REQUIRE(window_log2 >= 0 && window_log2 <= 31, "window_log2 must be 0..31, got %d", window_log2);
  HI3D_REQUIRE(n_f >= 0 && n_f < (int64_t(1) << 31) - 1, "bad fine row count");
  if (n_c == 0) return HI3D_OK;
  HI3D_REQUIRE(down && workspace && order && down_sorted, "null pointer argument");
  HI3D_REQUIRE(workspace_bytes >= need, "workspace too small: %lld < %lld bytes", static_cast<long long>(workspace_bytes),
               static_cast<long long>(need));
  const int64_t slab = align_up(n_c * 4, 256);
  char* w = static_cast<char*>(workspace);
  auto* k0 = reinterpret_cast<uint32_t*>(w);
  auto* k1 = reinterpret_cast<uint32_t*>(w + slab);
  auto* r0 = reinterpret_cast<int32_t*>(w + 2 * slab);
  auto* r1 = reinterpret_cast<int32_t*>(w + 3 * slab);
  const dim3 grid(static_cast<unsigned>(ceil_div(n_c, 256)));
  hipLaunchKernelGGL(up_keys_kernel, grid, dim3(256), 0, stream, down, n_c, n_f, static_cast<int>(window_log2), k0, r0);
  int window_bits = 0;
  while (window_bits < 31 - window_log2 && (int64_t(1) << (window_bits + window_log2)) < n_c) ++window_bits;
  HI3D_HIP_CHECK(radix::sort_pairs(w + 4 * slab, workspace_bytes - 4 * slab, k0, k1, r0, r1, n_c, 0,
                                   std::min(32, 8 + window_bits), stream));
  const int64_t npad = ceil_div(n_c, kUpParents) * kUpParents;
  hipLaunchKernelGGL(up_order_kernel, dim3(static_cast<unsigned>(ceil_div(npad, 256))), dim3(256), 0, stream, r0, down,
                     n_c, n_f, npad, order, down_sorted);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

int hi3d_stride2_up_conv_sorted(const void* in, int64_t n_c, int32_t cin, const void* weight, const void* bias,
                                int32_t cout, const int32_t* order, const int32_t* down_sorted, int64_t n_f,
                                int32_t dtype, void* out, void* stream) {
  int rc = up_check(cin, cout, dtype, n_c, n_f);
  if (rc != HI3D_OK) return rc;
  if (n_c == 0 || n_f == 0) return HI3D_OK;
  HI3D_REQUIRE(in && weight && order && down_sorted && out, "null pointer argument");
  HI3D_REQUIRE(((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(weight) |
                 reinterpret_cast<uintptr_t>(out)) & 15) == 0,
               "input, weight and output must be 16-byte aligned");
  UpArgs a{static_cast<const char*>(in), static_cast<const char*>(weight), bias, down_sorted, order,
           static_cast<char*>(out), n_c, n_f, ceil_div(n_c, kUpParents), static_cast<uint32_t>(n_f * cout * 2)};
  hipStream_t s = as_stream(stream);
  if (dtype == HI3D_BF16) return dispatch_up<__bf16, true>(a, cin, s);
  return dispatch_up<_Float16, true>(a, cin, s);
}

}  // extern "C"
