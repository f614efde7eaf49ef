// W8A8 int8 linear on gfx950: per-token quantiser (optionally signed-H64 rotated) and an
// int8 MFMA GEMM with int32 accumulators and the dequant + bias epilogue fused.
//
// Reference: src/hi3d_mac/mlx_backend/w8a8.py — signs :16-18, _QUANT :25-58,
// _GEMM :61-80, quantize_activation :95-102, linear :105-119.
#include "common.h"
#include "conv_tile.h"

namespace hi3d {
namespace {

// ------------------------------------------------------------------ quantiser --
// One wave per row. Pass p covers columns [512p, 512p + 512): lane l holds the 8
// consecutive columns 512p + 8l .. +7, i.e. positions 8(l%8) .. +7 of 64-column block
// 8p + l/8. Hadamard butterflies run over position bits 0..5 in increasing order, the
// same order as the reference's lane shuffles (bits 0..4) followed by its u/v combine
// (bit 5), so every intermediate value is the same IEEE fp32 operation:
//   pair (L, H) differing in bit d -> (L + H, L - H); the last stage also scales by 1/8.
// Position bits 0..2 live in registers, bits 3..5 are lane bits 0..2 (xor shuffles).
template <int NP, bool kRotate>
__global__ __launch_bounds__(256) void quant_kernel(const _Float16* __restrict__ x, int64_t m, int k,
                                                    const float* __restrict__ signs, int8_t* __restrict__ q,
                                                    float* __restrict__ scale) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= m) return;
  const _Float16* xr = x + row * k;
  float v[NP][8];
  float maximum = 0.0f;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int c0 = p * 512 + lane * 8;
    const bool ok = c0 < k;
    f16x8 h = {};
    if (ok) h = *reinterpret_cast<const f16x8*>(xr + c0);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[p][e] = static_cast<float>(h[e]);
    if (kRotate) {
      if (ok) {
        const float4 s0 = *reinterpret_cast<const float4*>(signs + c0);
        const float4 s1 = *reinterpret_cast<const float4*>(signs + c0 + 4);
        v[p][0] *= s0.x; v[p][1] *= s0.y; v[p][2] *= s0.z; v[p][3] *= s0.w;
        v[p][4] *= s1.x; v[p][5] *= s1.y; v[p][6] *= s1.z; v[p][7] *= s1.w;
      }
      // position bits 0, 1, 2 (in registers)
#pragma unroll
      for (int d = 1; d < 8; d <<= 1) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (e & d) continue;
          const float lo = v[p][e], hi = v[p][e + d];
          v[p][e] = lo + hi;
          v[p][e + d] = lo - hi;
        }
      }
      // position bits 3, 4 (lane bits 0, 1)
#pragma unroll
      for (int d = 1; d < 4; d <<= 1) {
        const bool upper = (lane & d) != 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float other = __shfl_xor(v[p][e], d, 64);
          v[p][e] = upper ? other - v[p][e] : v[p][e] + other;
        }
      }
      // position bit 5 (lane bit 2) with the 1/8 normalisation
      {
        const bool upper = (lane & 4) != 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float other = __shfl_xor(v[p][e], 4, 64);
          v[p][e] = upper ? (other - v[p][e]) * 0.125f : (v[p][e] + other) * 0.125f;
        }
      }
    }
    if (ok) {
#pragma unroll
      for (int e = 0; e < 8; ++e) maximum = fmaxf(maximum, fabsf(v[p][e]));
    }
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) maximum = fmaxf(maximum, __shfl_xor(maximum, d, 64));
  const float s = fmaxf(maximum, 1e-8f) / 127.0f;
  if (lane == 0) scale[row] = s;
  int8_t* qr = q + row * k;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int c0 = p * 512 + lane * 8;
    if (c0 >= k) continue;
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float r = __builtin_rintf(v[p][e] / s);
      r = fminf(fmaxf(r, -127.0f), 127.0f);
      const uint32_t b = static_cast<uint32_t>(static_cast<int32_t>(r)) & 0xffu;
      if (e < 4) lo |= b << (8 * e);
      else hi |= b << (8 * (e - 4));
    }
    *reinterpret_cast<uint2*>(qr + c0) = make_uint2(lo, hi);
  }
}

// -------------------------------------------------------------------- GEMM --
// C[m, n] = sum_k A[m, k] * W[n, k] on int8 MFMA 32x32x32 with int32 accumulators.
// Workgroup tile BM x BN, 4 waves in a 2x2 grid, K-blocks of 128 bytes double-buffered
// through LDS in the shared swizzled layout.
template <int BM, int BN>
__global__ __launch_bounds__(256) void w8a8_gemm_kernel(const int8_t* __restrict__ qa, const float* __restrict__ sa,
                                                        const int8_t* __restrict__ w, const float* __restrict__ sw,
                                                        const _Float16* __restrict__ bias, int64_t m, int n, int k,
                                                        _Float16* __restrict__ out, int32_t* __restrict__ acc_out,
                                                        int64_t mtiles, int ntiles) {
#pragma clang fp contract(off)
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int MB = WM / 32, NB = WN / 32;
  constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128;
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int PIPE = 2 * STAGE;
  constexpr int EPI = BM * BN * 2;
  constexpr int SMEM = PIPE > EPI ? PIPE : EPI;
  constexpr int AL = BM / 32, BL = BN / 32;
  __shared__ __attribute__((aligned(16))) char smem[SMEM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  // column tiles innermost: consecutive items share the A rows (L2 reuse in one XCD)
  const int64_t item = xcd_remap(blockIdx.x, static_cast<int64_t>(gridDim.x));
  const int64_t mt = item / ntiles;
  const int nt = static_cast<int>(item - mt * ntiles);
  const int64_t m0 = mt * BM;
  const int n0 = nt * BN;

  const int chunks = k >> 4;
  const int S = (chunks + 7) >> 3;
  const int ld_row = tid >> 3, ld_chunk = tid & 7;
  const u32x4 zero = {0u, 0u, 0u, 0u};
  u32x4 ra[AL], rb[BL];
  int ls = 0;
  auto load = [&]() {
    const int c = ls * 8 + ld_chunk;
    const bool cok = c < chunks;
#pragma unroll
    for (int i = 0; i < AL; ++i) {
      const int64_t r = m0 + ld_row + 32 * i;
      ra[i] = (cok && r < m) ? *reinterpret_cast<const u32x4*>(qa + r * k + c * 16) : zero;
    }
#pragma unroll
    for (int j = 0; j < BL; ++j) {
      const int r = n0 + ld_row + 32 * j;
      rb[j] = (cok && r < n) ? *reinterpret_cast<const u32x4*>(w + static_cast<int64_t>(r) * k + c * 16) : zero;
    }
    ++ls;
  };
  auto store = [&](int buf) {
    char* A = smem + buf * STAGE;
    char* B = A + A_BYTES;
#pragma unroll
    for (int i = 0; i < AL; ++i) *reinterpret_cast<u32x4*>(A + lds_offset(ld_row + 32 * i, ld_chunk)) = ra[i];
#pragma unroll
    for (int j = 0; j < BL; ++j) *reinterpret_cast<u32x4*>(B + lds_offset(ld_row + 32 * j, ld_chunk)) = rb[j];
  };
  i32x16 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mb][nb][v] = 0;
  auto compute = [&](int buf) {
    const char* A = smem + buf * STAGE;
    const char* B = A + A_BYTES;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c = 2 * g + (lane >> 5);
      u32x4 af[MB], bf[NB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        af[mb] = *reinterpret_cast<const u32x4*>(A + lds_offset(wm * WM + mb * 32 + (lane & 31), c));
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        bf[nb] = *reinterpret_cast<const u32x4*>(B + lds_offset(wn * WN + nb * 32 + (lane & 31), c));
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          acc[mb][nb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, af[mb]),
                                                               __builtin_bit_cast(i32x4, bf[nb]), acc[mb][nb], 0, 0, 0);
    }
  };
  if (S > 0) {
    load();
    store(0);
    __syncthreads();
    for (int s = 0; s < S; ++s) {
      const bool more = s + 1 < S;
      if (more) load();
      compute(s & 1);
      if (more) store((s + 1) & 1);
      __syncthreads();
    }
  }
  // epilogue: fp16(((float)acc * sa) * sw + (float)bias), staged in LDS for 16-byte stores
  _Float16* C = reinterpret_cast<_Float16*>(smem);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int j = wn * WN + nb * 32 + (lane & 31);
    const int col = n0 + j;
    const bool cok = col < n;
    const float swc = cok ? sw[col] : 0.0f;
    const float bc = (cok && bias != nullptr) ? static_cast<float>(bias[col]) : 0.0f;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int i = wm * WM + mb * 32 + acc_row(lane, v);
        const int64_t row = m0 + i;
        const float sar = row < m ? sa[row] : 0.0f;
        const float prod = static_cast<float>(acc[mb][nb][v]) * sar;
        const float y = prod * swc + bc;
        C[i * BN + j] = static_cast<_Float16>(y);
        if (acc_out != nullptr && cok && row < m) acc_out[row * n + col] = acc[mb][nb][v];
      }
    }
  }
  __syncthreads();
  constexpr int CPR = BN / 8;
  for (int q = tid; q < BM * CPR; q += 256) {
    const int i = q / CPR, cc = q - (q / CPR) * CPR;
    const int64_t row = m0 + i;
    const int col = n0 + cc * 8;
    if (row >= m || col >= n) continue;
    const u32x4 v = *reinterpret_cast<const u32x4*>(C + i * BN + cc * 8);
    if (col + 8 <= n && (n & 7) == 0) {
      *reinterpret_cast<u32x4*>(out + row * n + col) = v;
    } else {
      const _Float16* pv = reinterpret_cast<const _Float16*>(&v);
      for (int e = 0; e < 8 && col + e < n; ++e) out[row * n + col + e] = pv[e];
    }
  }
}

template <int NP>
void launch_quant(const _Float16* x, int64_t m, int k, const float* signs, int8_t* q, float* s, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(ceil_div(m, 4)));
  if (signs) hipLaunchKernelGGL((quant_kernel<NP, true>), grid, dim3(256), 0, stream, x, m, k, signs, q, s);
  else hipLaunchKernelGGL((quant_kernel<NP, false>), grid, dim3(256), 0, stream, x, m, k, signs, q, s);
}

}  // namespace
}  // namespace hi3d

using namespace hi3d;

extern "C" {

int hi3d_w8a8_quantize(const void* x, int64_t m, int32_t k, const float* signs, int8_t* q, float* scale,
                       void* stream_) {
  hipStream_t stream = as_stream(stream_);
  HI3D_REQUIRE(m >= 0 && k > 0, "bad sizes");
  HI3D_REQUIRE(k % 8 == 0, "width must be a multiple of 8 (got %d)", k);
  if (signs) HI3D_REQUIRE(k % 64 == 0, "signed H64 requires width divisible by 64");
  HI3D_REQUIRE(k <= 16384, "width above 16384 is not supported");
  if (m == 0) return HI3D_OK;
  HI3D_REQUIRE(x && q && scale, "null pointer argument");
  HI3D_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(q) & 7) == 0,
               "x must be 16-byte and q 8-byte aligned");
  const _Float16* xh = static_cast<const _Float16*>(x);
  const int passes = (k + 511) / 512;
  if (passes <= 1) launch_quant<1>(xh, m, k, signs, q, scale, stream);
  else if (passes <= 2) launch_quant<2>(xh, m, k, signs, q, scale, stream);
  else if (passes <= 4) launch_quant<4>(xh, m, k, signs, q, scale, stream);
  else if (passes <= 8) launch_quant<8>(xh, m, k, signs, q, scale, stream);
  else if (passes <= 16) launch_quant<16>(xh, m, k, signs, q, scale, stream);
  else launch_quant<32>(xh, m, k, signs, q, scale, stream);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

int hi3d_w8a8_gemm(const int8_t* q, const float* sa, const int8_t* w, const float* sw, const void* bias, int64_t m,
                   int32_t n, int32_t k, void* out, int32_t* acc_out, void* stream_) {
  hipStream_t stream = as_stream(stream_);
  HI3D_REQUIRE(m >= 0 && n > 0 && k > 0, "bad sizes");
  HI3D_REQUIRE(k % 16 == 0, "k must be a multiple of 16 (got %d)", k);
  if (m == 0) return HI3D_OK;
  HI3D_REQUIRE(q && sa && w && sw && out, "null pointer argument");
  HI3D_REQUIRE(((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(out)) & 15) == 0,
               "q, w and out must be 16-byte aligned");
  constexpr int BM = 128, BN = 256;
  const int64_t mtiles = ceil_div(m, BM);
  const int ntiles = static_cast<int>(ceil_div(n, BN));
  const int64_t blocks = mtiles * ntiles;
  HI3D_REQUIRE(blocks < (int64_t(1) << 31), "problem too large");
  hipLaunchKernelGGL((w8a8_gemm_kernel<BM, BN>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, q, sa, w,
                     sw, static_cast<const _Float16*>(bias), m, n, k, static_cast<_Float16*>(out), acc_out, mtiles,
                     ntiles);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

}  // extern "C"
