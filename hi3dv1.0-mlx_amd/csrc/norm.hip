// LayerNorm (+ adaLN modulation) row kernel and the adaLN projection, fp16 rows.
//
// Reference: layer_norm_modulate (src/hi3d_mac/mlx_backend/kernels.py:162-237),
// LayerNorm32 (src/sparc3d/nn/norm.py:12-17), the W8A8 activation quantiser that
// follows a norm in the transformer block (src/hi3d_mac/mlx_backend/w8a8.py:25-58,
// 95-102; src/hi3d_mac/mlx_backend/transformer.py:548-549, 570-571, 575-577), the res-block modulation
// (src/sparc3d/models/transformers/sparc3d_transformer.py:132-144,
// src/hi3d_mac/mlx_backend/transformer.py:413-424).
#include "common.h"
#include "conv_tile.h"
#include "quant.h"
#include "rownorm.h"

namespace hi3d {
namespace {

// G lanes per row, CPL 8-element chunks per lane (chunk g + i G), held in registers;
// fp32 two-pass statistics; y = (x - mean) * inv [* w + b]; h = fp16(y); modulate
// h = fp16(fp16(h * scale) + shift) (two roundings, no FMA, modulate8); kSilu: h =
// silu(h) in fp16.
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
        o[e] = static_cast<_Float16>(f32_rounded(y));
      }
      if constexpr (modulate) o = modulate8(o, sv[i], hv[i]);
      if constexpr (kSilu) {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = silu_h(o[e]);
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
    _Float16 h = static_cast<_Float16>(f32_rounded(y));
    if (scale != nullptr) {
      const _Float16 p = static_cast<_Float16>(static_cast<float>(h) * static_cast<float>(scale[i]));
      h = static_cast<_Float16>(static_cast<float>(p) + static_cast<float>(shift[i]));
    }
    if (act == HI3D_ACT_SILU) h = silu_h(h);
    orow[i] = h;
  }
}

// Lane L's partner L ^ d (d a power of two up to 32, a constant after unrolling): DPP
// for 1 to 8, ds_swizzle's bit-mask mode (and 0x1F, or 0, xor 16) for 16 within each
// 32-lane half, ds_bpermute for 32. The same partners as __shfl_xor, so a reduction
// over them gives the same value.
__device__ __forceinline__ float lane_xor(float v, int d) {
  switch (d) {
    case 1: return dpp_xor1(v);
    case 2: return dpp_xor2(v);
    case 4: return dpp_xor4(v);
    case 8: return dpp_xor8(v);
    case 16: return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
    default: return __shfl_xor(v, d, 64);
  }
}

// LayerNorm (+ affine and / or modulate) followed by the per-token int8 quantiser, in one
// pass: the row's fp16 output h is computed exactly as ln_kernel computes it (the same
// lanes, chunks, summation order and reduction partners) and is not stored; its values
// (times the multipliers and rotated by the block Hadamard when kRotate) are quantised
// as quant_kernel quantises a stored row, so q and the scale are bitwise those of the
// two kernels in sequence.
// Lanes and chunks as in ln_kernel: G lanes per row, chunk g + i G of 8 columns on
// lane g. A 64-column block is the chunks i of 8 consecutive lanes (G >= 8 when
// rotating), column 8 (g & 7) + e of the block on lane g, element e: the butterflies
// run over bits 0..2 in registers, then over bits 3..5 across lanes g ^ 1, ^ 2, ^ 4, the
// same pairs in the same increasing bit order as the quantiser, each pair (L, H) ->
// (L + H, L - H) (the upper lane adds the negated own value: L + (-H) = L - H).
// The multipliers, scale and shift sit in LDS (registers are what bounds the waves per
// SIMD here); the affine vectors are loaded into registers once. Rows past the end run
// the arithmetic (every lane of a row group takes part in the lane moves) and store
// nothing.
template <int G, int CPL, bool kAffine, bool kModulate, bool kRotate>
__global__ __launch_bounds__(256) void ln_quant_kernel(const _Float16* __restrict__ x, int64_t rows, int c, float eps,
                                                       const float* __restrict__ weight, const float* __restrict__ bias,
                                                       const _Float16* __restrict__ scale,
                                                       const _Float16* __restrict__ shift,
                                                       const float* __restrict__ signs, int8_t* __restrict__ q,
                                                       float* __restrict__ q_scale) {
#pragma clang fp contract(off)
  static_assert(!kRotate || G >= 8, "a rotated 64-column block spans 8 lanes");
  // LDS: the c multipliers (fp32) when rotating, then scale and shift (fp16) when modulating
  extern __shared__ __attribute__((aligned(16))) float lds_vec[];
  float* const mult = lds_vec;
  _Float16* const s_scale = reinterpret_cast<_Float16*>(lds_vec + (kRotate ? c : 0));
  _Float16* const s_shift = s_scale + c;
  constexpr int RPB = 256 / G;
  const int t = threadIdx.x;
  const int g = t % G;
  const int chunks = c >> 3;
  if constexpr (kRotate) {
    for (int i = t * 4; i < c; i += 1024) *reinterpret_cast<float4*>(mult + i) = *reinterpret_cast<const float4*>(signs + i);
  }
  if constexpr (kModulate) {
    for (int i = t * 8; i < c; i += 2048) {
      *reinterpret_cast<f16x8*>(s_scale + i) = *reinterpret_cast<const f16x8*>(scale + i);
      *reinterpret_cast<f16x8*>(s_shift + i) = *reinterpret_cast<const f16x8*>(shift + i);
    }
  }
  if constexpr (kRotate || kModulate) __syncthreads();
  f32x4 wv[kAffine ? CPL : 1][2], bv[kAffine ? CPL : 1][2];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int ch = g + i * G;
    if (ch >= chunks) continue;
    if constexpr (kAffine) {
      wv[i][0] = *reinterpret_cast<const f32x4*>(weight + ch * 8);
      wv[i][1] = *reinterpret_cast<const f32x4*>(weight + ch * 8 + 4);
      bv[i][0] = *reinterpret_cast<const f32x4*>(bias + ch * 8);
      bv[i][1] = *reinterpret_cast<const f32x4*>(bias + ch * 8 + 4);
    }
  }
  // the signs of the cross-lane butterfly terms: the lane with the bit set computes L - H
  const float up1 = (g & 1) ? -1.0f : 1.0f, up2 = (g & 2) ? -1.0f : 1.0f, up4 = (g & 4) ? -1.0f : 1.0f;
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
      if (live && ch < chunks) h = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(xr + ch * 8));
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[i][e] = static_cast<float>(h[e]);
        sum += v[i][e];
      }
    }
#pragma unroll
    for (int d = G / 2; d >= 1; d >>= 1) sum += lane_xor(sum, d);
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
    for (int d = G / 2; d >= 1; d >>= 1) sq += lane_xor(sq, d);
    const float inv = 1.0f / sqrtf(sq / static_cast<float>(c) + eps);
    // the norm's fp16 output, as a float (times the multiplier when rotating); zeros in
    // chunks past the row, which leave the maximum unchanged
    float maximum = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int ch = g + i * G;
      const bool ok = ch < chunks;
      const int cl = (ok ? ch : 0) * 8;  // LDS column of the chunk
      f32x4 mv[2];
      f16x8 sv, hv;
      if constexpr (kRotate) {
        mv[0] = *reinterpret_cast<const f32x4*>(mult + cl);
        mv[1] = *reinterpret_cast<const f32x4*>(mult + cl + 4);
      }
      if constexpr (kModulate) {
        sv = *reinterpret_cast<const f16x8*>(s_scale + cl);
        hv = *reinterpret_cast<const f16x8*>(s_shift + cl);
      }
      f16x8 h;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float y = (v[i][e] - mean) * inv;
        if constexpr (kAffine) y = y * wv[i][e >> 2][e & 3] + bv[i][e >> 2][e & 3];
        h[e] = static_cast<_Float16>(f32_rounded(y));
      }
      if constexpr (kModulate) h = modulate8(h, sv, hv);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float u = ok ? static_cast<float>(h[e]) : 0.0f;
        if constexpr (kRotate) u *= mv[e >> 2][e & 3];
        v[i][e] = u;
      }
      if constexpr (kRotate) {
#pragma unroll
        for (int d = 1; d < 8; d <<= 1) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            if (e & d) continue;
            const float lo = v[i][e], hi = v[i][e + d];
            v[i][e] = lo + hi;
            v[i][e + d] = lo - hi;
          }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = dpp_xor1(v[i][e]) + v[i][e] * up1;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = dpp_xor2(v[i][e]) + v[i][e] * up2;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = dpp_xor4(v[i][e]) + v[i][e] * up4;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) maximum = fmaxf(maximum, fabsf(v[i][e]));
    }
#pragma unroll
    for (int d = G / 2; d >= 1; d >>= 1) maximum = fmaxf(maximum, lane_xor(maximum, d));
    float s;
    const QuantDivisor dv = quant_divisor<kRotate>(maximum, s);
    if (dv.fast) {
#pragma unroll
      for (int i = 0; i < CPL; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = quant_div(v[i][e], dv.t, dv.r);
    } else {
#pragma unroll
      for (int i = 0; i < CPL; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = v[i][e] / dv.t;
    }
    if (!live) continue;
    if (g == 0) q_scale[row] = s;
    int8_t* qr = q + row * c;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int ch = g + i * G;
      if (ch >= chunks) continue;
      *reinterpret_cast<uint2*>(qr + ch * 8) = make_uint2(quant_pack4(v[i][0], v[i][1], v[i][2], v[i][3]),
                                                          quant_pack4(v[i][4], v[i][5], v[i][6], v[i][7]));
    }
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

template <int G, int CPL, bool kAffine, bool kModulate, bool kRotate>
void launch_ln_quant_kernel(const _Float16* x, int64_t rows, int c, float eps, const float* w, const float* b,
                            const _Float16* sc, const _Float16* sh, const float* signs, int8_t* q, float* qs,
                            hipStream_t stream) {
  constexpr int RPB = 256 / G;
  const size_t lds = static_cast<size_t>(c) * ((kRotate ? sizeof(float) : 0) + (kModulate ? 2 * sizeof(_Float16) : 0));
  const int cus = compute_units();
  const int64_t groups = ceil_div(rows, RPB);
  const int64_t cap = static_cast<int64_t>(cus > 0 ? cus : 256) * 16;  // a few strides per block
  const dim3 grid(static_cast<unsigned>(groups < cap ? groups : cap));
  hipLaunchKernelGGL((ln_quant_kernel<G, CPL, kAffine, kModulate, kRotate>), grid, dim3(256), lds, stream, x, rows, c,
                     eps, w, b, sc, sh, signs, q, qs);
}

template <int G, int CPL, bool kRotate>
void launch_ln_quant(const _Float16* x, int64_t rows, int c, float eps, const float* w, const float* b,
                     const _Float16* sc, const _Float16* sh, const float* signs, int8_t* q, float* qs,
                     hipStream_t stream) {
  if (w != nullptr && sc != nullptr)
    launch_ln_quant_kernel<G, CPL, true, true, kRotate>(x, rows, c, eps, w, b, sc, sh, signs, q, qs, stream);
  else if (w != nullptr)
    launch_ln_quant_kernel<G, CPL, true, false, kRotate>(x, rows, c, eps, w, b, sc, sh, signs, q, qs, stream);
  else if (sc != nullptr)
    launch_ln_quant_kernel<G, CPL, false, true, kRotate>(x, rows, c, eps, w, b, sc, sh, signs, q, qs, stream);
  else
    launch_ln_quant_kernel<G, CPL, false, false, kRotate>(x, rows, c, eps, w, b, sc, sh, signs, q, qs, stream);
}

// Lanes per row as launch_ln_width, at least 8 (a rotated block spans 8 lanes).
template <bool kRotate>
void launch_ln_quant_width(const _Float16* x, int64_t rows, int c, float eps, const float* w, const float* b,
                           const _Float16* sc, const _Float16* sh, const float* signs, int8_t* q, float* qs,
                           hipStream_t stream) {
  const int chunks = c / 8;
  if (chunks <= 8) launch_ln_quant<8, 1, kRotate>(x, rows, c, eps, w, b, sc, sh, signs, q, qs, stream);
  else if (chunks <= 16) launch_ln_quant<8, 2, kRotate>(x, rows, c, eps, w, b, sc, sh, signs, q, qs, stream);
  else if (chunks <= 32) launch_ln_quant<8, 4, kRotate>(x, rows, c, eps, w, b, sc, sh, signs, q, qs, stream);
  else if (chunks <= 64) launch_ln_quant<16, 4, kRotate>(x, rows, c, eps, w, b, sc, sh, signs, q, qs, stream);
  else if (chunks <= 128) launch_ln_quant<32, 4, kRotate>(x, rows, c, eps, w, b, sc, sh, signs, q, qs, stream);
  else if (chunks <= 256) launch_ln_quant<64, 4, kRotate>(x, rows, c, eps, w, b, sc, sh, signs, q, qs, stream);
  else launch_ln_quant<64, 8, kRotate>(x, rows, c, eps, w, b, sc, sh, signs, q, qs, stream);
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

int hi3d_layer_norm_quantize(const void* x, int64_t rows, int32_t c, float eps, const float* weight, const float* bias,
                             const void* scale, const void* shift, const float* signs, int8_t* q, float* q_scale,
                             void* stream) {
  HI3D_REQUIRE(rows >= 0 && c > 0, "bad sizes");
  HI3D_REQUIRE((weight == nullptr) == (bias == nullptr), "weight and bias must be given together");
  HI3D_REQUIRE((scale == nullptr) == (shift == nullptr), "scale and shift must be given together");
  HI3D_REQUIRE(c % 8 == 0, "width must be a multiple of 8 (got %d)", c);
  if (signs) HI3D_REQUIRE(c % 64 == 0, "signed H64 requires width divisible by 64");
  HI3D_REQUIRE(c <= 4096, "width above 4096 is not supported (got %d)", c);
  if (rows == 0) return HI3D_OK;
  HI3D_REQUIRE(x && q && q_scale, "null pointer argument");
  const uintptr_t vec = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight) |
                        reinterpret_cast<uintptr_t>(bias) | reinterpret_cast<uintptr_t>(scale) |
                        reinterpret_cast<uintptr_t>(shift) | reinterpret_cast<uintptr_t>(signs);
  HI3D_REQUIRE((vec & 15) == 0 && (reinterpret_cast<uintptr_t>(q) & 7) == 0,
               "rows, per-channel vectors and multipliers must be 16-byte aligned, q 8-byte aligned");
  const auto* xh = static_cast<const _Float16*>(x);
  const auto* sc = static_cast<const _Float16*>(scale);
  const auto* sh = static_cast<const _Float16*>(shift);
  if (signs) launch_ln_quant_width<true>(xh, rows, c, eps, weight, bias, sc, sh, signs, q, q_scale, as_stream(stream));
  else launch_ln_quant_width<false>(xh, rows, c, eps, weight, bias, sc, sh, signs, q, q_scale, as_stream(stream));
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
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
