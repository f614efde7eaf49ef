// Per-token int8 quantiser arithmetic shared by the W8A8 quantiser (w8a8.hip) and the
// fused LayerNorm + quantise kernel (norm.hip).
//
// Reference: src/hi3d_mac/mlx_backend/w8a8.py:25-58 (_QUANT).
#pragma once

#include "conv_tile.h"

namespace hi3d {

// Lane moves: the value of lane L ^ d. DPP controls: quad_perm [1,0,3,2] (0xB1) = L ^ 1,
// [2,3,0,1] (0x4E) = L ^ 2, [3,2,1,0] (0x1B) = L ^ 3; row_half_mirror (0x141) = L ^ 7
// within 8 lanes; row_mirror (0x140) = L ^ 15 within 16 lanes.
template <int kCtrl>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, true));
}
__device__ __forceinline__ float dpp_xor1(float v) { return dpp_mov<0xB1>(v); }
__device__ __forceinline__ float dpp_xor2(float v) { return dpp_mov<0x4E>(v); }
__device__ __forceinline__ float dpp_xor4(float v) { return dpp_mov<0x1B>(dpp_mov<0x141>(v)); }  // (L ^ 7) ^ 3
__device__ __forceinline__ float dpp_xor8(float v) { return dpp_mov<0x141>(dpp_mov<0x140>(v)); }  // (L ^ 15) ^ 7

// Divisor of a row's values from the maximum of their magnitudes.
// Rotated rows hold the unscaled block-Hadamard sums, 8x the reference's values (which
// carry a final * 0.125): scaling by a power of two commutes with rounding away from the
// subnormal range, so t = fl(max(8 max|v|, 8e-8) / 127) is exactly 8 s for the
// reference's s = fl(max(max|v|, 1e-8) / 127), and v / t is the reference's quotient,
// the same real number. Unrotated rows: t = s.
// r is rcp(t) refined by one Newton step, for the division sequence of quant_div.
struct QuantDivisor {
  float t, r;
  bool fast;  // t finite: quant_div's sequence is the correctly rounded quotient
};

template <bool kRotated>
__device__ __forceinline__ QuantDivisor quant_divisor(float maximum, float& scale) {
#pragma clang fp contract(off)
  QuantDivisor d;
  if constexpr (kRotated) {
    d.t = fmaxf(maximum, 1e-8f * 8.0f) / 127.0f;  // 8 s
    scale = d.t * 0.125f;
  } else {
    d.t = fmaxf(maximum, 1e-8f) / 127.0f;
    scale = d.t;
  }
  d.fast = __builtin_isfinite(d.t);
  const float r0 = __builtin_amdgcn_rcpf(d.t);
  d.r = __builtin_fmaf(__builtin_fmaf(-d.t, r0, 1.0f), r0, r0);
  return d;
}

// a / t with the compiler's own correctly rounded f32 division sequence, its reciprocal
// refinement hoisted per row:  q = a r, e = a - t q, q1 = q + e r, e1 = a - t q1,
// a / t = q1 + e1 r (fma each). The full division's pre-scaling (v_div_scale) and
// fix-up only act when the quotient is below 2^-126 or a below 2^-103 (t is at least
// 8e-8 / 127 and |a| / t at most 127), where both round to 0. For finite t only.
__device__ __forceinline__ float quant_div(float a, float t, float r) {
#pragma clang fp contract(off)
  const float q0 = a * r;
  const float q1 = __builtin_fmaf(__builtin_fmaf(-t, q0, a), r, q0);
  return __builtin_fmaf(__builtin_fmaf(-t, q1, a), r, q1);
}

// Four quotients to int8 codes (round half to even, clamp to +-127), packed low first.
__device__ __forceinline__ uint32_t quant_pack4(float a, float b, float c, float d) {
  const float v[4] = {a, b, c, d};
  uint32_t packed = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float rr = fminf(fmaxf(__builtin_rintf(v[e]), -127.0f), 127.0f);
    packed |= (static_cast<uint32_t>(static_cast<int32_t>(rr)) & 0xffu) << (8 * e);
  }
  return packed;
}

}  // namespace hi3d
