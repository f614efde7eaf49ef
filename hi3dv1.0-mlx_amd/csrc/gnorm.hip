// GroupNorm statistics and the GroupNorm + swish activation in front of the VAE decoder's
// sparse convolutions.
//
// Reference: SparconvVAEDecoderMLX.group_stats / conv_gn_swish / resnet
// (src/hi3d_mac/mlx_backend/vae.py:141-218) and gather_group_norm_swish
// (src/hi3d_mac/mlx_backend/kernels.py:240-296).
//
// The reference activates each gathered neighbour row while it assembles the GEMM's
// [rows, 27 C] input block. The gather-MFMA convolution here moves rows straight from
// HBM into LDS, so the activation runs once per row instead: swish(GN(x)) [n, C] in one
// elementwise pass (27 times fewer elements than the gathered block), then the
// convolution gathers it. Absent neighbours still read zeros, the convolution's padding
// applied to the activated features as in the reference.
#include "common.h"
#include "conv_tile.h"

namespace hi3d {
namespace {

constexpr int kStatsBlocksPerCu = 4;

// 8 consecutive elements of x as fp32.
template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    const u32x4 raw = *reinterpret_cast<const u32x4*>(p);
    const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = static_cast<float>(e[i]);
  } else {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = a[i];
      v[i + 4] = b[i];
    }
  }
}

template <typename T>
__device__ __forceinline__ void store8(T* p, const float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    u32x4 raw;
    T* e = reinterpret_cast<T*>(&raw);
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = static_cast<T>(v[i]);
    *reinterpret_cast<u32x4*>(p) = raw;
  } else {
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
  }
}

// Column sums of x [n, c] (c % 8 == 0, c <= 2048): thread t owns the 8 channels
// 8 (t % tc) .. +7 (tc = c / 8) of rows t / tc + rpi i (rpi = 256 / tc rows per step);
// block b takes steps b, b + B, ... and writes its fp32 sums of x and x x per channel to
// partial[b][2][c].
template <typename T>
__global__ __launch_bounds__(256) void colsum_kernel(const T* __restrict__ x, int64_t n, int c,
                                                     float* __restrict__ partial) {
#pragma clang fp contract(off)
  __shared__ float red[2][256 * 8];
  const int tc = c >> 3, rpi = 256 / tc;
  const int t = threadIdx.x, cc = t % tc, r0 = t / tc;
  float s1[8] = {}, s2[8] = {};
  if (r0 < rpi) {
    const int64_t step = static_cast<int64_t>(gridDim.x) * rpi;
    int64_t row = static_cast<int64_t>(blockIdx.x) * rpi + r0;
    // four rows' loads in flight, then their sums in row order
    for (; row + 3 * step < n; row += 4 * step) {
      float v[4][8];
#pragma unroll
      for (int u = 0; u < 4; ++u) load8(x + (row + u * step) * c + cc * 8, v[u]);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          s1[e] += v[u][e];
          s2[e] += v[u][e] * v[u][e];
        }
    }
    for (; row < n; row += step) {
      float v[8];
      load8(x + row * c + cc * 8, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        s1[e] += v[e];
        s2[e] += v[e] * v[e];
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    red[0][t * 8 + e] = s1[e];
    red[1][t * 8 + e] = s2[e];
  }
  __syncthreads();
  for (int ch = t; ch < c; ch += 256) {
    const int q = ch >> 3, e = ch & 7;
    float a = 0.0f, b = 0.0f;
    for (int r = 0; r < rpi; ++r) {
      a += red[0][(r * tc + q) * 8 + e];
      b += red[1][(r * tc + q) * 8 + e];
    }
    partial[(static_cast<int64_t>(blockIdx.x) * 2) * c + ch] = a;
    partial[(static_cast<int64_t>(blockIdx.x) * 2 + 1) * c + ch] = b;
  }
}

// Per-channel sums of the block partials in fp64, in a fixed order: a block takes 16
// channels, its thread t sums every 16th partial from t / 16 for channel t % 16, then
// the 16 slices are added in order. sums[0][c] = S1, sums[1][c] = S2.
__global__ __launch_bounds__(256) void colsum_finish_kernel(const float* __restrict__ partial, int blocks, int c,
                                                            double* __restrict__ sums) {
  __shared__ double red[2][16][16];
  const int t = threadIdx.x, j = t & 15, sl = t >> 4;
  const int ch = blockIdx.x * 16 + j;
  double a = 0.0, b = 0.0;
  if (ch < c) {
    for (int k = sl; k < blocks; k += 16) {
      a += partial[(static_cast<int64_t>(k) * 2) * c + ch];
      b += partial[(static_cast<int64_t>(k) * 2 + 1) * c + ch];
    }
  }
  red[0][sl][j] = a;
  red[1][sl][j] = b;
  __syncthreads();
  if (sl == 0 && ch < c) {
    double sa = 0.0, sb = 0.0;
    for (int i = 0; i < 16; ++i) {
      sa += red[0][i][j];
      sb += red[1][i][j];
    }
    sums[ch] = sa;
    sums[c + ch] = sb;
  }
}

// Per group of `width` consecutive channels: mean = S1 / (count + eps),
// var = S2 / (count + eps) - mean^2, inv = 1 / sqrt(var + eps) with count = n width;
// written per channel.
__global__ __launch_bounds__(256) void group_finish_kernel(const double* __restrict__ sums, int64_t n, int c,
                                                           int groups, float eps, float* __restrict__ mean,
                                                           float* __restrict__ inv) {
  const int g = blockIdx.x * 256 + threadIdx.x;
  if (g >= groups) return;
  const int width = c / groups;
  const double count = static_cast<double>(n) * width + static_cast<double>(eps);
  double a = 0.0, b = 0.0;
  for (int j = 0; j < width; ++j) {
    a += sums[g * width + j];
    b += sums[c + g * width + j];
  }
  const double m = a / count;
  const double var = b / count - m * m;
  const float mf = static_cast<float>(m);
  const float iv = 1.0f / sqrtf(static_cast<float>(var) + eps);
  for (int j = 0; j < width; ++j) {
    mean[g * width + j] = mf;
    inv[g * width + j] = iv;
  }
}

// u = ((x - mean) inv) weight + bias and u sigmoid(u) in fp32, the sigmoid in the
// reference's form e = 1 / (1 + exp(|u|)), sigmoid = u < 0 ? e : 1 - e. exp and the
// reciprocal use the hardware's exp2 and rcp (about 2 ulp; the reference computes this
// activation under Metal's fast math, and its tests gate it at 1e-5 / 2e-3).
struct GnParams8 {
  float m[8], iv[8], w[8], b[8];
};

__device__ __forceinline__ void gn_load8(GnParams8& p, const float* __restrict__ mean, const float* __restrict__ inv,
                                         const float* __restrict__ weight, const float* __restrict__ bias, int ch) {
  load8(mean + ch, p.m);
  load8(inv + ch, p.iv);
  load8(weight + ch, p.w);
  load8(bias + ch, p.b);
}

__device__ __forceinline__ void gn_swish8(float (&v)[8], const GnParams8& p) {
#pragma clang fp contract(off)
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float u = ((v[e] - p.m[e]) * p.iv[e]) * p.w[e] + p.b[e];
    const float s = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(fabsf(u) * 1.44269504088896341f));
    v[e] = u * (u < 0.0f ? s : 1.0f - s);
  }
}

__device__ __forceinline__ void gn_swish8(float (&v)[8], const float* __restrict__ mean, const float* __restrict__ inv,
                                          const float* __restrict__ weight, const float* __restrict__ bias, int ch) {
  GnParams8 p;
  gn_load8(p, mean, inv, weight, bias, ch);
  gn_swish8(v, p);
}

// out [n, c] = swish(GN(x)) in Tout; 8 channels per thread, grid-stride.
template <typename Tin, typename Tout>
__global__ __launch_bounds__(256) void gn_swish_kernel(const Tin* __restrict__ x, int64_t n, int c,
                                                       const float* __restrict__ mean, const float* __restrict__ inv,
                                                       const float* __restrict__ weight,
                                                       const float* __restrict__ bias, Tout* __restrict__ out) {
  const int tc = c >> 3;
  const int64_t total = n * tc;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (stride % tc == 0) {
    // the thread's channel group is the same in every step: its parameters load once
    const int ch = static_cast<int>(first % tc) * 8;
    GnParams8 p;
    gn_load8(p, mean, inv, weight, bias, ch);
    for (int64_t i = first; i < total; i += stride) {
      const int64_t row = i / tc;
      float v[8];
      load8(x + row * c + ch, v);
      gn_swish8(v, p);
      store8(out + row * c + ch, v);
    }
    return;
  }
  for (int64_t i = first; i < total; i += stride) {
    const int64_t row = i / tc;
    const int ch = static_cast<int>(i - row * tc) * 8;
    float v[8];
    load8(x + row * c + ch, v);
    gn_swish8(v, mean, inv, weight, bias, ch);
    store8(out + row * c + ch, v);
  }
}

// out [j, c] = swish(GN(x))[table[j]] (zeros where table[j] is outside [0, n)) for the
// j entries of a [rows, kvol] table, i.e. the [rows, kvol c] block.
template <typename Tin, typename Tout>
__global__ __launch_bounds__(256) void gather_gn_swish_kernel(const Tin* __restrict__ x, int64_t n, int c,
                                                              const int32_t* __restrict__ table, int64_t entries,
                                                              const float* __restrict__ mean,
                                                              const float* __restrict__ inv,
                                                              const float* __restrict__ weight,
                                                              const float* __restrict__ bias, Tout* __restrict__ out) {
  const int tc = c >> 3;
  const int64_t total = entries * tc;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t j = i / tc;
    const int ch = static_cast<int>(i - j * tc) * 8;
    const int32_t r = table[j];
    float v[8];
    if (static_cast<uint64_t>(static_cast<uint32_t>(r)) < static_cast<uint64_t>(n)) {
      load8(x + static_cast<int64_t>(r) * c + ch, v);
      gn_swish8(v, mean, inv, weight, bias, ch);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = 0.0f;
    }
    store8(out + j * c + ch, v);
  }
}

int stats_blocks(int64_t n, int c) {
  const int rpi = 256 / (c >> 3);
  const int64_t steps = ceil_div(n, static_cast<int64_t>(rpi));
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(steps, int64_t(compute_units()) * kStatsBlocksPerCu)));
}

// partial sums [blocks][2][c] fp32, then the per-channel fp64 sums [2][c]
int64_t partial_bytes(int64_t n, int c) { return align_up(static_cast<int64_t>(stats_blocks(n, c)) * 2 * c * 4, 256); }
int64_t stats_workspace(int64_t n, int c) { return partial_bytes(n, c) + static_cast<int64_t>(2) * c * 8; }

int grid_for(int64_t items) {
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(ceil_div(items, int64_t(256)), int64_t(compute_units()) * 16)));
}

template <typename Tin>
int launch_gn_swish(const Tin* x, int64_t n, int c, const float* mean, const float* inv, const float* w,
                    const float* b, void* out, int32_t out_dtype, hipStream_t s) {
  const dim3 grid(grid_for(n * (c >> 3)));
  switch (out_dtype) {
    case HI3D_F16: hipLaunchKernelGGL((gn_swish_kernel<Tin, _Float16>), grid, dim3(256), 0, s, x, n, c, mean, inv, w, b, static_cast<_Float16*>(out)); break;
    case HI3D_BF16: hipLaunchKernelGGL((gn_swish_kernel<Tin, __bf16>), grid, dim3(256), 0, s, x, n, c, mean, inv, w, b, static_cast<__bf16*>(out)); break;
    case HI3D_F32: hipLaunchKernelGGL((gn_swish_kernel<Tin, float>), grid, dim3(256), 0, s, x, n, c, mean, inv, w, b, static_cast<float*>(out)); break;
    default: HI3D_REQUIRE(false, "unsupported output dtype %d", out_dtype);
  }
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

template <typename Tin>
int launch_gather_gn_swish(const Tin* x, int64_t n, int c, const int32_t* table, int64_t entries, const float* mean,
                           const float* inv, const float* w, const float* b, void* out, int32_t out_dtype,
                           hipStream_t s) {
  const dim3 grid(grid_for(entries * (c >> 3)));
  switch (out_dtype) {
    case HI3D_F16: hipLaunchKernelGGL((gather_gn_swish_kernel<Tin, _Float16>), grid, dim3(256), 0, s, x, n, c, table, entries, mean, inv, w, b, static_cast<_Float16*>(out)); break;
    case HI3D_BF16: hipLaunchKernelGGL((gather_gn_swish_kernel<Tin, __bf16>), grid, dim3(256), 0, s, x, n, c, table, entries, mean, inv, w, b, static_cast<__bf16*>(out)); break;
    case HI3D_F32: hipLaunchKernelGGL((gather_gn_swish_kernel<Tin, float>), grid, dim3(256), 0, s, x, n, c, table, entries, mean, inv, w, b, static_cast<float*>(out)); break;
    default: HI3D_REQUIRE(false, "unsupported output dtype %d", out_dtype);
  }
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

int check_rows(const void* x, int32_t dtype, int32_t c) {
  HI3D_REQUIRE(dtype == HI3D_F16 || dtype == HI3D_BF16 || dtype == HI3D_F32, "unsupported dtype %d", dtype);
  HI3D_REQUIRE(c > 0 && c % 8 == 0 && c <= 2048, "channels must be a multiple of 8, at most 2048 (got %d)", c);
  HI3D_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15) == 0, "rows must be 16-byte aligned");
  return HI3D_OK;
}

}  // namespace
}  // namespace hi3d

using namespace hi3d;

extern "C" {

int hi3d_group_stats_workspace(int64_t n, int32_t c, int64_t* bytes) {
  HI3D_REQUIRE(bytes != nullptr, "null pointer argument");
  HI3D_REQUIRE(n >= 0 && c > 0 && c % 8 == 0 && c <= 2048, "bad sizes");
  *bytes = stats_workspace(n, c);
  return HI3D_OK;
}

int hi3d_group_stats(const void* x, int32_t dtype, int64_t n, int32_t c, int32_t groups, float eps, void* workspace,
                     int64_t workspace_bytes, float* mean, float* inv, void* stream_) {
  hipStream_t s = as_stream(stream_);
  if (const int rc = check_rows(x, dtype, c); rc != HI3D_OK) return rc;
  HI3D_REQUIRE(n >= 0, "negative row count");
  HI3D_REQUIRE(groups > 0 && c % groups == 0, "channels (%d) must split into %d groups", c, groups);
  HI3D_REQUIRE((x || n == 0) && workspace && mean && inv, "null pointer argument");
  const int blocks = stats_blocks(n, c);
  HI3D_REQUIRE(workspace_bytes >= stats_workspace(n, c), "workspace too small");
  float* partial = static_cast<float*>(workspace);
  double* sums = reinterpret_cast<double*>(static_cast<char*>(workspace) + partial_bytes(n, c));
  switch (dtype) {
    case HI3D_F16: hipLaunchKernelGGL((colsum_kernel<_Float16>), dim3(blocks), dim3(256), 0, s, static_cast<const _Float16*>(x), n, c, partial); break;
    case HI3D_BF16: hipLaunchKernelGGL((colsum_kernel<__bf16>), dim3(blocks), dim3(256), 0, s, static_cast<const __bf16*>(x), n, c, partial); break;
    default: hipLaunchKernelGGL((colsum_kernel<float>), dim3(blocks), dim3(256), 0, s, static_cast<const float*>(x), n, c, partial); break;
  }
  HI3D_LAUNCH_CHECK();
  hipLaunchKernelGGL(colsum_finish_kernel, dim3(static_cast<unsigned>(ceil_div(c, 16))), dim3(256), 0, s, partial, blocks, c,
                     sums);
  HI3D_LAUNCH_CHECK();
  hipLaunchKernelGGL(group_finish_kernel, dim3(static_cast<unsigned>(ceil_div(groups, 256))), dim3(256), 0, s, sums, n, c,
                     groups, eps, mean, inv);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

int hi3d_gn_swish(const void* x, int32_t dtype, int64_t n, int32_t c, const float* mean, const float* inv,
                  const float* weight, const float* bias, void* out, int32_t out_dtype, void* stream_) {
  hipStream_t s = as_stream(stream_);
  if (const int rc = check_rows(x, dtype, c); rc != HI3D_OK) return rc;
  if (n == 0) return HI3D_OK;
  HI3D_REQUIRE(mean && inv && weight && bias && out, "null pointer argument");
  HI3D_REQUIRE(((reinterpret_cast<uintptr_t>(mean) | reinterpret_cast<uintptr_t>(inv) | reinterpret_cast<uintptr_t>(weight) |
                 reinterpret_cast<uintptr_t>(bias) | reinterpret_cast<uintptr_t>(out)) & 15) == 0,
               "vectors and output must be 16-byte aligned");
  switch (dtype) {
    case HI3D_F16: return launch_gn_swish(static_cast<const _Float16*>(x), n, c, mean, inv, weight, bias, out, out_dtype, s);
    case HI3D_BF16: return launch_gn_swish(static_cast<const __bf16*>(x), n, c, mean, inv, weight, bias, out, out_dtype, s);
    default: return launch_gn_swish(static_cast<const float*>(x), n, c, mean, inv, weight, bias, out, out_dtype, s);
  }
}

int hi3d_gather_gn_swish(const void* x, int32_t dtype, int64_t n, int32_t c, const int32_t* table, int64_t entries,
                         const float* mean, const float* inv, const float* weight, const float* bias, void* out,
                         int32_t out_dtype, void* stream_) {
  hipStream_t s = as_stream(stream_);
  if (const int rc = check_rows(x, dtype, c); rc != HI3D_OK) return rc;
  if (entries == 0) return HI3D_OK;
  HI3D_REQUIRE(table && mean && inv && weight && bias && out, "null pointer argument");
  HI3D_REQUIRE(((reinterpret_cast<uintptr_t>(mean) | reinterpret_cast<uintptr_t>(inv) | reinterpret_cast<uintptr_t>(weight) |
                 reinterpret_cast<uintptr_t>(bias) | reinterpret_cast<uintptr_t>(out)) & 15) == 0,
               "vectors and output must be 16-byte aligned");
  switch (dtype) {
    case HI3D_F16: return launch_gather_gn_swish(static_cast<const _Float16*>(x), n, c, table, entries, mean, inv, weight, bias, out, out_dtype, s);
    case HI3D_BF16: return launch_gather_gn_swish(static_cast<const __bf16*>(x), n, c, table, entries, mean, inv, weight, bias, out, out_dtype, s);
    default: return launch_gather_gn_swish(static_cast<const float*>(x), n, c, table, entries, mean, inv, weight, bias, out, out_dtype, s);
  }
}

}  // extern "C"
