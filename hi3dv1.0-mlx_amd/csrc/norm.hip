// LayerNorm (+ adaLN modulation) row kernel and the adaLN projection, fp16 rows.
//
// Reference: layer_norm_modulate (src/hi3d_mac/mlx_backend/kernels.py:162-237),
// LayerNorm32 (src/sparc3d/nn/norm.py:12-17), the res-block modulation
// (src/sparc3d/models/transformers/sparc3d_transformer.py:132-144,
// src/hi3d_mac/mlx_backend/transformer.py:413-424).
#include "common.h"
#include "conv_tile.h"

namespace hi3d {
namespace {

// SiLU of an fp16 value as the reference's fp16 ``x * sigmoid(x)``
// (src/hi3d_mac/mlx_backend/transformer.py:172-173): the sigmoid rounded to fp16, then
// the product rounded to fp16.
__device__ __forceinline__ _Float16 silu_h(_Float16 h) {
#pragma clang fp contract(off)
  const float x = static_cast<float>(h);
  const _Float16 sig = static_cast<_Float16>(1.0f / (1.0f + __expf(-x)));
  return static_cast<_Float16>(x * static_cast<float>(sig));
}

// G lanes per row, CPL 8-element chunks per lane (chunk g + i G), held in registers;
// fp32 two-pass statistics; y = (x - mean) * inv [* w + b]; h = fp16(y); modulate
// h = fp16(fp16(h * scale) + shift) (two roundings, no FMA); kSilu: h = silu(h) in fp16.
// The per-channel vectors of a lane's chunks are loaded once; blocks stride over groups
// of 256 / G rows.
template <int G, int CPL, bool kAffine, bool kModulate, bool kSilu = false>
__global__ __launch_bounds__(256) void ln_kernel(const _Float16* __restrict__ x, int64_t rows, int c, float eps,
                                                 const float* __restrict__ weight, const float* __restrict__ bias,
                                                 const _Float16* __restrict__ scale,
                                                 const _Float16* __restrict__ shift, _Float16* __restrict__ out) {
#pragma clang fp contract(off)
  constexpr int RPB = 256 / G;  // rows per block per step
  const int t = threadIdx.x;
  const int g = t % G;
  const int chunks = c >> 3;
  constexpr bool affine = kAffine, modulate = kModulate;
  f32x4 wv[kAffine ? CPL : 1][2], bv[kAffine ? CPL : 1][2];
  f16x8 sv[kModulate ? CPL : 1], hv[kModulate ? CPL : 1];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int ch = g + i * G;
    const bool ok = ch < chunks;
    if constexpr (affine) {
      if (!ok) continue;
      wv[i][0] = *reinterpret_cast<const f32x4*>(weight + ch * 8);
      wv[i][1] = *reinterpret_cast<const f32x4*>(weight + ch * 8 + 4);
      bv[i][0] = *reinterpret_cast<const f32x4*>(bias + ch * 8);
      bv[i][1] = *reinterpret_cast<const f32x4*>(bias + ch * 8 + 4);
    }
    if constexpr (modulate) {
      if (!ok) continue;
      sv[i] = *reinterpret_cast<const f16x8*>(scale + ch * 8);
      hv[i] = *reinterpret_cast<const f16x8*>(shift + ch * 8);
    }
  }
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * RPB; base < rows; base += static_cast<int64_t>(gridDim.x) * RPB) {
    const int64_t row = base + t / G;
    const bool live = row < rows;
    const _Float16* xr = x + (live ? row : 0) * c;
    float v[CPL][8];
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int ch = g + i * G;
      f16x8 h = {};
      // rows are read and written once: nontemporal, so the stream does not evict what
      // the convolution reads next (config 5: 0.89 -> 0.82 ms, the block 15.91 -> 15.80 ms)
      if (live && ch < chunks) h = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(xr + ch * 8));
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[i][e] = static_cast<float>(h[e]);
        sum += v[i][e];
      }
    }
#pragma unroll
    for (int d = G / 2; d >= 1; d >>= 1) sum += __shfl_xor(sum, d, 64);
    const float mean = sum / static_cast<float>(c);
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int ch = g + i * G;
      if (ch < chunks) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = v[i][e] - mean;
          sq += d * d;
        }
      }
    }
#pragma unroll
    for (int d = G / 2; d >= 1; d >>= 1) sq += __shfl_xor(sq, d, 64);
    const float inv = 1.0f / sqrtf(sq / static_cast<float>(c) + eps);
    if (!live) continue;
    _Float16* orow = out + row * c;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int ch = g + i * G;
      if (ch >= chunks) continue;
      f16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float y = (v[i][e] - mean) * inv;
        if constexpr (affine) y = y * wv[i][e >> 2][e & 3] + bv[i][e >> 2][e & 3];
        _Float16 h = static_cast<_Float16>(y);
        if constexpr (modulate) {
          const _Float16 p = static_cast<_Float16>(static_cast<float>(h) * static_cast<float>(sv[i][e]));
          h = static_cast<_Float16>(static_cast<float>(p) + static_cast<float>(hv[i][e]));
        }
        if constexpr (kSilu) h = silu_h(h);
        o[e] = h;
      }
      __builtin_nontemporal_store(o, reinterpret_cast<f16x8*>(orow + ch * 8));
    }
  }
}

// Any width: one wave per row, three passes over the row in global memory.
__global__ __launch_bounds__(256) void ln_generic_kernel(const _Float16* __restrict__ x, int64_t rows, int c, float eps,
                                                         const float* __restrict__ weight,
                                                         const float* __restrict__ bias,
                                                         const _Float16* __restrict__ scale,
                                                         const _Float16* __restrict__ shift, int act,
                                                         _Float16* __restrict__ out) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const _Float16* xr = x + row * c;
  float sum = 0.0f;
  for (int i = lane; i < c; i += 64) sum += static_cast<float>(xr[i]);
  for (int d = 32; d >= 1; d >>= 1) sum += __shfl_xor(sum, d, 64);
  const float mean = sum / static_cast<float>(c);
  float sq = 0.0f;
  for (int i = lane; i < c; i += 64) {
    const float d = static_cast<float>(xr[i]) - mean;
    sq += d * d;
  }
  for (int d = 32; d >= 1; d >>= 1) sq += __shfl_xor(sq, d, 64);
  const float inv = 1.0f / sqrtf(sq / static_cast<float>(c) + eps);
  _Float16* orow = out + row * c;
  for (int i = lane; i < c; i += 64) {
    float y = (static_cast<float>(xr[i]) - mean) * inv;
    if (weight != nullptr) y = y * weight[i] + bias[i];
    _Float16 h = static_cast<_Float16>(y);
    if (scale != nullptr) {
      const _Float16 p = static_cast<_Float16>(static_cast<float>(h) * static_cast<float>(scale[i]));
      h = static_cast<_Float16>(static_cast<float>(p) + static_cast<float>(shift[i]));
    }
    if (act == HI3D_ACT_SILU) h = silu_h(h);
    orow[i] = h;
  }
}

// One wave per output feature: y = W . cond' + b (fp32), then the fp16 (1 + scale) and
// shift halves.
__global__ __launch_bounds__(256) void adaln_kernel(const float* __restrict__ w, const float* __restrict__ b,
                                                    const float* __restrict__ cond, int n_out, int n_in, int apply_silu,
                                                    _Float16* __restrict__ scale1p, _Float16* __restrict__ shift) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int j = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (j >= n_out) return;
  const float* wr = w + static_cast<int64_t>(j) * n_in;
  float acc = 0.0f;
  for (int i = lane; i < n_in; i += 64) {
    float ci = cond[i];
    if (apply_silu) ci = ci / (1.0f + expf(-ci));
    acc += wr[i] * ci;
  }
  for (int d = 32; d >= 1; d >>= 1) acc += __shfl_xor(acc, d, 64);
  if (lane != 0) return;
  const float y = acc + (b != nullptr ? b[j] : 0.0f);
  const int half = n_out / 2;
  const _Float16 yh = static_cast<_Float16>(y);
  if (j < half) scale1p[j] = static_cast<_Float16>(1.0f + static_cast<float>(yh));
  else shift[j - half] = yh;
}

template <int G, int CPL, bool kSilu>
void launch_ln(const _Float16* x, int64_t rows, int c, float eps, const float* w, const float* b, const _Float16* sc,
               const _Float16* sh, _Float16* out, hipStream_t stream) {
  constexpr int RPB = 256 / G;
  const int64_t groups = ceil_div(rows, RPB);
  const int cus = compute_units();
  const int64_t cap = static_cast<int64_t>(cus > 0 ? cus : 256) * 16;  // a few strides per block
  const dim3 grid(static_cast<unsigned>(groups < cap ? groups : cap));
  if (w != nullptr && sc != nullptr)
    hipLaunchKernelGGL((ln_kernel<G, CPL, true, true, kSilu>), grid, dim3(256), 0, stream, x, rows, c, eps, w, b, sc, sh,
                       out);
  else if (w != nullptr)
    hipLaunchKernelGGL((ln_kernel<G, CPL, true, false, kSilu>), grid, dim3(256), 0, stream, x, rows, c, eps, w, b, sc,
                       sh, out);
  else if (sc != nullptr)
    hipLaunchKernelGGL((ln_kernel<G, CPL, false, true, kSilu>), grid, dim3(256), 0, stream, x, rows, c, eps, w, b, sc,
                       sh, out);
  else
    hipLaunchKernelGGL((ln_kernel<G, CPL, false, false, kSilu>), grid, dim3(256), 0, stream, x, rows, c, eps, w, b, sc,
                       sh, out);
}

template <bool kSilu>
void launch_ln_width(const _Float16* xh, int64_t rows, int c, float eps, const float* weight, const float* bias,
                     const _Float16* sc, const _Float16* sh, _Float16* o, hipStream_t stream) {
  const int chunks = c / 8;
  if (chunks <= 4) launch_ln<4, 1, kSilu>(xh, rows, c, eps, weight, bias, sc, sh, o, stream);
  else if (chunks <= 8) launch_ln<8, 1, kSilu>(xh, rows, c, eps, weight, bias, sc, sh, o, stream);
  else if (chunks <= 16) launch_ln<8, 2, kSilu>(xh, rows, c, eps, weight, bias, sc, sh, o, stream);
  else if (chunks <= 32) launch_ln<8, 4, kSilu>(xh, rows, c, eps, weight, bias, sc, sh, o, stream);
  else if (chunks <= 64) launch_ln<16, 4, kSilu>(xh, rows, c, eps, weight, bias, sc, sh, o, stream);
  else if (chunks <= 128) launch_ln<32, 4, kSilu>(xh, rows, c, eps, weight, bias, sc, sh, o, stream);
  else if (chunks <= 256) launch_ln<64, 4, kSilu>(xh, rows, c, eps, weight, bias, sc, sh, o, stream);
  else launch_ln<64, 8, kSilu>(xh, rows, c, eps, weight, bias, sc, sh, o, stream);
}

int layer_norm(const void* x, int64_t rows, int32_t c, float eps, const float* weight, const float* bias,
               const void* scale, const void* shift, int32_t act, void* out, hipStream_t stream) {
  HI3D_REQUIRE(rows >= 0 && c > 0, "bad sizes");
  HI3D_REQUIRE((weight == nullptr) == (bias == nullptr), "weight and bias must be given together");
  HI3D_REQUIRE((scale == nullptr) == (shift == nullptr), "scale and shift must be given together");
  HI3D_REQUIRE(act == HI3D_ACT_NONE || act == HI3D_ACT_SILU, "unknown activation %d", act);
  if (rows == 0) return HI3D_OK;
  HI3D_REQUIRE(x && out, "null pointer argument");
  const auto* xh = static_cast<const _Float16*>(x);
  const auto* sc = static_cast<const _Float16*>(scale);
  const auto* sh = static_cast<const _Float16*>(shift);
  auto* o = static_cast<_Float16*>(out);
  const uintptr_t vec = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
                        reinterpret_cast<uintptr_t>(weight) | reinterpret_cast<uintptr_t>(bias) |
                        reinterpret_cast<uintptr_t>(scale) | reinterpret_cast<uintptr_t>(shift);
  if (c % 8 == 0 && (vec & 15) == 0 && c / 8 <= 64 * 8) {
    if (act == HI3D_ACT_SILU) launch_ln_width<true>(xh, rows, c, eps, weight, bias, sc, sh, o, stream);
    else launch_ln_width<false>(xh, rows, c, eps, weight, bias, sc, sh, o, stream);
  } else {
    hipLaunchKernelGGL(ln_generic_kernel, dim3(static_cast<unsigned>(ceil_div(rows, 4))), dim3(256), 0, stream, xh, rows,
                       c, eps, weight, bias, sc, sh, act, o);
  }
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

}  // namespace
}  // namespace hi3d

using namespace hi3d;

extern "C" {

int hi3d_layer_norm_modulate(const void* x, int64_t rows, int32_t c, float eps, const float* weight, const float* bias,
                             const void* scale, const void* shift, void* out, void* stream) {
  return layer_norm(x, rows, c, eps, weight, bias, scale, shift, HI3D_ACT_NONE, out, as_stream(stream));
}

int hi3d_layer_norm_act(const void* x, int64_t rows, int32_t c, float eps, const float* weight, const float* bias,
                        const void* scale, const void* shift, int32_t act, void* out, void* stream) {
  return layer_norm(x, rows, c, eps, weight, bias, scale, shift, act, out, as_stream(stream));
}

int hi3d_adaln_projection(const float* w, const float* b, const float* cond, int32_t n_out, int32_t n_in,
                          int32_t apply_silu, void* scale1p, void* shift, void* stream_) {
  hipStream_t stream = as_stream(stream_);
  HI3D_REQUIRE(n_out > 0 && n_out % 2 == 0 && n_in > 0, "n_out must be even and positive, n_in positive");
  HI3D_REQUIRE(w && cond && scale1p && shift, "null pointer argument");
  hipLaunchKernelGGL(adaln_kernel, dim3(static_cast<unsigned>(ceil_div(n_out, 4))), dim3(256), 0, stream, w, b, cond,
                     n_out, n_in, apply_silu, static_cast<_Float16*>(scale1p), static_cast<_Float16*>(shift));
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

}  // extern "C"
