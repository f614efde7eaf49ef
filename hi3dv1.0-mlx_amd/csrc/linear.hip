// Row-wise linear layer on fp16 rows with the residual epilogue of the convolutions: the
// res block's `linear(h) + skip_connection(x)` as one pass over the rows.
//
// Reference: SparseResBlock3d.forward's last line (src/sparc3d/models/transformers/
// sparc3d_transformer.py:143-144) and its MLX form _resblock_tail
// (src/hi3d_mac/mlx_backend/transformer.py:426-437).
#include "common.h"
#include "conv_tile.h"

namespace hi3d {
namespace {

// out[n, cout] = fp16(x W^T + bias), then with a residual fp16(out + residual): the
// rounding points of the gather convolution's epilogue (the product rounded once, the
// residual added to that fp16 value and rounded again), and its MFMA sequence
// (v_mfma_f32_32x32x16_f16, weights as the first operand, K-groups of 16 in order), so
// the bits equal those of the convolution over the one-offset identity plan.
//
// A workgroup has one wave per 64-channel slice of the output (cout / 64 <= 4 waves); each
// wave keeps its slice's weights in registers for the whole launch (2 blocks of 32
// channels x KG K-groups of 16, 16 bytes per lane each). Workgroups walk 32-row tiles:
//  * the tile's rows reach LDS once for all waves: each thread loads its 16-byte chunks
//    of the next tile into registers while the current one is computed, and writes them
//    into the other of two LDS buffers (rows of 128 or 256 bytes, chunk c of row r at
//    c ^ (r & 7): the fragment reads of 8 consecutive rows hit 8 distinct bank groups);
//    one barrier per tile (a buffer is rewritten two tiles later, after every wave has
//    passed the next barrier);
//  * each wave reads its fragments (row lane % 32, K half lane / 32), runs 2 x KG MFMAs,
//    and stages its fp32 accumulators (32 rows x 64 channels) in its own LDS region;
//  * it reads them back row-contiguous (a lane: 8 channels of one row, 8 lanes per row),
//    adds the bias, rounds, adds the residual and stores: 16-byte accesses, 8 rows per
//    instruction (the residual's loads are issued before the MFMAs).
// Rows past n read row n - 1 and store nothing. The residual may alias the output (each
// element is read, then written, by the same lane).
template <int KG, int S>
__global__ __launch_bounds__(64 * S) void dense_linear_kernel(const _Float16* __restrict__ x, int64_t n, int cin,
                                                            const _Float16* __restrict__ w,
                                                            const _Float16* __restrict__ bias, int cout,
                                                            const _Float16* residual, _Float16* out, int64_t tiles) {
  constexpr int XCH = 2 * KG;                  // 16-byte chunks of an input row
  constexpr int XS = XCH <= 8 ? 128 : 256;     // LDS row stride of the input tile
  constexpr int XBUF = 32 * XS;                // one input tile
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int nthreads = 64 * S;
  const int c0 = wave * 64;  // this wave's channel slice
  char* const stage = smem + 2 * XBUF + wave * (32 * 256);
  const int half = lane >> 5, r32 = lane & 31;

  u32x4 wf[2][KG];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int g = 0; g < KG; ++g)
      wf[b][g] = *reinterpret_cast<const u32x4*>(w + static_cast<int64_t>(c0 + 32 * b + r32) * cin + 16 * g + 8 * half);
  // epilogue layout: lane -> row (lane / 8) + 8 i, channels c0 + 8 (lane % 8) + 0..7
  const int er = lane >> 3, ec = (lane & 7) * 8;
  float bv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) bv[e] = bias != nullptr ? static_cast<float>(bias[c0 + ec + e]) : 0.0f;

  // this thread's chunks of an input tile: i = tid + k * nthreads, row i / XCH, chunk i % XCH
  constexpr int kChunks = (32 * XCH + nthreads - 1) / nthreads;
  u32x4 xr[kChunks];
  auto load_tile = [&](int64_t t) {
#pragma unroll
    for (int k = 0; k < kChunks; ++k) {
      const int i = tid + k * nthreads;
      if (i < 32 * XCH) {
        int64_t row = t * 32 + i / XCH;
        row = row < n ? row : n - 1;
        xr[k] = *reinterpret_cast<const u32x4*>(x + row * cin + (i % XCH) * 8);
      }
    }
  };
  auto store_tile = [&](char* buf) {
#pragma unroll
    for (int k = 0; k < kChunks; ++k) {
      const int i = tid + k * nthreads;
      if (i < 32 * XCH) {
        const int row = i / XCH, c = i % XCH;
        *reinterpret_cast<u32x4*>(buf + row * XS + ((c ^ (row & 7)) << 4)) = xr[k];
      }
    }
  };

  int64_t t = blockIdx.x;
  if (t < tiles) load_tile(t);
  for (int buf = 0; t < tiles; t += gridDim.x, buf ^= 1) {
    char* const xb = smem + buf * XBUF;
    store_tile(xb);
    const int64_t tn = t + gridDim.x;
    // the residual of this tile (before the next tile's loads, so waiting for it does
    // not wait for them)
    u32x4 rv[4];
    if (residual != nullptr) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        int64_t row = t * 32 + er + 8 * i;
        row = row < n ? row : n - 1;
        rv[i] = *reinterpret_cast<const u32x4*>(residual + row * cout + c0 + ec);
      }
    }
    if (tn < tiles) load_tile(tn);
    __syncthreads();
    f32x16 acc[2] = {};
#pragma unroll
    for (int g = 0; g < KG; ++g) {
      const int c = 2 * g + half;
      const u32x4 xf = *reinterpret_cast<const u32x4*>(xb + r32 * XS + ((c ^ (r32 & 7)) << 4));
#pragma unroll
      for (int b = 0; b < 2; ++b) Mfma<_Float16>::run(wf[b][g], xf, acc[b]);
    }
    // stage: row r32, channels 32 b + 8 q + 4 half + 0..3 = fp32 chunk 8 b + 2 q + half
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int j = 8 * b + 2 * q + half;
        const f32x4 v = {acc[b][4 * q], acc[b][4 * q + 1], acc[b][4 * q + 2], acc[b][4 * q + 3]};
        *reinterpret_cast<f32x4*>(stage + r32 * 256 + ((j ^ (r32 & 7)) << 4)) = v;
      }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = er + 8 * i;
      const int j0 = ec >> 2;  // fp32 chunks j0, j0 + 1
      const f32x4 lo = *reinterpret_cast<const f32x4*>(stage + row * 256 + ((j0 ^ (row & 7)) << 4));
      const f32x4 hi = *reinterpret_cast<const f32x4*>(stage + row * 256 + (((j0 + 1) ^ (row & 7)) << 4));
      const int64_t orow = t * 32 + row;
      _Float16 h[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        h[e] = static_cast<_Float16>(lo[e] + bv[e]);
        h[e + 4] = static_cast<_Float16>(hi[e] + bv[e + 4]);
      }
      u32x4 packed;
      __builtin_memcpy(&packed, h, 16);
      if (residual != nullptr) packed = add_chunk<_Float16>(packed, rv[i]);
      if (orow < n) *reinterpret_cast<u32x4*>(out + orow * cout + c0 + ec) = packed;
    }
  }
}

template <int KG, int S>
void launch_dense_linear_s(const _Float16* x, int64_t n, int cin, const _Float16* w, const _Float16* bias, int cout,
                           const _Float16* residual, _Float16* out, int64_t tiles, int64_t grid, hipStream_t stream) {
  const size_t lds = 2 * 32 * (2 * KG <= 8 ? 128 : 256) + static_cast<size_t>(S) * 32 * 256;
  hipLaunchKernelGGL((dense_linear_kernel<KG, S>), dim3(static_cast<unsigned>(grid)), dim3(64 * S), lds, stream, x, n,
                     cin, w, bias, cout, residual, out, tiles);
}

template <int KG>
void launch_dense_linear(const _Float16* x, int64_t n, int cin, const _Float16* w, const _Float16* bias, int cout,
                         const _Float16* residual, _Float16* out, int64_t tiles, int64_t grid, hipStream_t stream) {
  switch (cout / 64) {
    case 1: launch_dense_linear_s<KG, 1>(x, n, cin, w, bias, cout, residual, out, tiles, grid, stream); break;
    case 2: launch_dense_linear_s<KG, 2>(x, n, cin, w, bias, cout, residual, out, tiles, grid, stream); break;
    case 3: launch_dense_linear_s<KG, 3>(x, n, cin, w, bias, cout, residual, out, tiles, grid, stream); break;
    default: launch_dense_linear_s<KG, 4>(x, n, cin, w, bias, cout, residual, out, tiles, grid, stream); break;
  }
}

}  // namespace
}  // namespace hi3d

using namespace hi3d;

extern "C" {

int hi3d_dense_linear(const void* x, int64_t n, int32_t cin, const void* weight, const void* bias, int32_t cout,
                      const void* residual, void* out, void* stream_) {
  hipStream_t stream = as_stream(stream_);
  HI3D_REQUIRE(n >= 0, "bad sizes");
  HI3D_REQUIRE(cin > 0 && cin % 16 == 0 && cin <= 128, "cin must be a multiple of 16 up to 128 (got %d)", cin);
  HI3D_REQUIRE(cout > 0 && cout % 64 == 0 && cout <= 256, "cout must be 64, 128, 192 or 256 (got %d)", cout);
  if (n == 0) return HI3D_OK;
  HI3D_REQUIRE(x && weight && out, "null pointer argument");
  const uintptr_t vec = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight) |
                        reinterpret_cast<uintptr_t>(residual) | reinterpret_cast<uintptr_t>(out);
  HI3D_REQUIRE((vec & 15) == 0 && (reinterpret_cast<uintptr_t>(bias) & 1) == 0,
               "rows and weights must be 16-byte aligned");
  const int cus = compute_units();
  HI3D_REQUIRE(cus > 0, "cannot query the compute unit count");
  // persistent workgroups: about 8 waves per CU (two per SIMD at this register count)
  const int slices = cout / 64;
  const int64_t tiles = ceil_div(n, 32);
  int64_t grid = static_cast<int64_t>(cus) * (8 / slices);
  if (grid > tiles) grid = tiles;
  const auto* xh = static_cast<const _Float16*>(x);
  const auto* wh = static_cast<const _Float16*>(weight);
  const auto* bh = static_cast<const _Float16*>(bias);
  const auto* rh = static_cast<const _Float16*>(residual);
  auto* oh = static_cast<_Float16*>(out);
  switch (cin / 16) {
    case 1: launch_dense_linear<1>(xh, n, cin, wh, bh, cout, rh, oh, tiles, grid, stream); break;
    case 2: launch_dense_linear<2>(xh, n, cin, wh, bh, cout, rh, oh, tiles, grid, stream); break;
    case 3: launch_dense_linear<3>(xh, n, cin, wh, bh, cout, rh, oh, tiles, grid, stream); break;
    case 4: launch_dense_linear<4>(xh, n, cin, wh, bh, cout, rh, oh, tiles, grid, stream); break;
    case 5: launch_dense_linear<5>(xh, n, cin, wh, bh, cout, rh, oh, tiles, grid, stream); break;
    case 6: launch_dense_linear<6>(xh, n, cin, wh, bh, cout, rh, oh, tiles, grid, stream); break;
    case 7: launch_dense_linear<7>(xh, n, cin, wh, bh, cout, rh, oh, tiles, grid, stream); break;
    default: launch_dense_linear<8>(xh, n, cin, wh, bh, cout, rh, oh, tiles, grid, stream); break;
  }
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

}  // extern "C"
