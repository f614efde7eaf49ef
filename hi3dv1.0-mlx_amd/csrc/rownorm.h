// fp16 row-normalisation steps shared by the LayerNorm kernels (norm.hip) and the
// convolution epilogue that applies the res block's second norm (conv.hip).
//
// Reference: layer_norm_modulate (src/hi3d_mac/mlx_backend/kernels.py:162-237) and the
// fp16 SiLU of the res blocks (src/hi3d_mac/mlx_backend/transformer.py:172-173).
#pragma once

#include "conv_tile.h"

namespace hi3d {

// SiLU of an fp16 value as the reference's fp16 ``x * sigmoid(x)``
// (src/hi3d_mac/mlx_backend/transformer.py:172-173): the sigmoid rounded to fp16, then
// the product rounded to fp16. The sigmoid runs through the hardware exp2 and
// reciprocal (~1 ulp each in fp32); its fp16 rounding differs from that of the exact
// sigmoid in about one value in 10^4. The product of two fp16 values is exact in fp32,
// so the native fp16 multiply rounds it as the fp32 product rounded to fp16 does.
__device__ __forceinline__ _Float16 silu_h(_Float16 h) {
#pragma clang fp contract(off)
  const float x = static_cast<float>(h);
  const _Float16 sig = static_cast<_Float16>(__builtin_amdgcn_rcpf(1.0f + __expf(-x)));
  return h * sig;
}

// The norm's f32 value, rounded to f32 and kept as such before its conversion to fp16:
// without this the compiler folds fp16((x - mean) * inv) into one mixed-precision FMA
// (v_fma_mixlo_f16), which rounds the exact product to fp16 once instead of to f32 and
// then to fp16, and differs from the reference in rare last bits.
__device__ __forceinline__ float f32_rounded(float y) {
  asm("" : "+v"(y));
  return y;
}

// fp16(fp16(h * scale) + shift) on 8 columns with native fp16 multiplies and adds (no
// FMA). The reference rounds each step through fp32; a product of two fp16 values is
// exact in fp32, and fp32 carries more than twice fp16's precision plus two bits, so
// rounding through fp32 and rounding once give the same fp16 results.
__device__ __forceinline__ f16x8 modulate8(f16x8 h, f16x8 scale, f16x8 shift) {
#pragma clang fp contract(off)
  const f16x8 p = h * scale;
  return p + shift;
}

}  // namespace hi3d
