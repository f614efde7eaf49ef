// W8A8 int8 linear on gfx950: per-token quantiser (optionally signed-H64 rotated) and an
// int8 MFMA GEMM with int32 accumulators and the dequant + bias epilogue fused.
//
// Reference: src/hi3d_mac/mlx_backend/w8a8.py — signs :16-18, _QUANT :25-58,
// _GEMM :61-80, quantize_activation :95-102, linear :105-119.
#include <type_traits>

#include "common.h"
#include "conv_tile.h"
#include "quant.h"

namespace hi3d {
namespace {

// ------------------------------------------------------------------ quantiser --
// One wave per row, grid-stride over rows, the next row's fp16 data loaded while the
// current one is computed. Pass p covers columns [1024p, 1024p + 1024): lane l holds the
// 16 consecutive columns 1024p + 16l .. +15, i.e. positions 16(l%4) .. +15 of 64-column
// block 16p + l/4. Hadamard butterflies run over position bits 0..5 in increasing
// order, the same order as the reference's lane shuffles (bits 0..4) followed by its
// u/v combine (bit 5):  pair (L, H) differing in bit d -> (L + H, L - H).
// Bits 0..3 live in registers, bits 4 and 5 are lane bits 0 and 1 (quad DPP moves).
// The reference scales the last stage by 1/8; here the values stay unscaled (8x theirs)
// and the 1/8 moves into the scale (quant_divisor). Quantisation divides with the
// compiler's own correctly rounded f32 division sequence, its reciprocal refinement
// hoisted per row (quant_div); rows with a non-finite scale use the full division.
// The multipliers (signs) sit in LDS, loaded once per workgroup.
constexpr int kQuantCols = 1024;  // columns per pass

template <int NP, bool kRotate, bool kFull>
__global__ __launch_bounds__(256) void quant_kernel(const _Float16* __restrict__ x, int64_t m, int k,
                                                    const float* __restrict__ signs, int8_t* __restrict__ q,
                                                    float* __restrict__ scale) {
#pragma clang fp contract(off)
  extern __shared__ __attribute__((aligned(16))) float mult[];  // k multipliers when rotating
  constexpr bool kHold = NP <= 8;      // row held in registers (else recomputed)
  constexpr bool kPrefetch = NP <= 4;  // and the next row's loads in flight meanwhile
  const int lane = threadIdx.x & 63;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 4;
  if constexpr (kRotate) {
    for (int i = threadIdx.x * 4; i < k; i += 1024)
      *reinterpret_cast<float4*>(mult + i) = *reinterpret_cast<const float4*>(signs + i);
    __syncthreads();
  }
  const float up1 = (lane & 1) ? -1.0f : 1.0f, up2 = (lane & 2) ? -1.0f : 1.0f;
  // loads are unconditional (straight-line code keeps the wait counts exact): chunks
  // past k load column 0 of the row and are zeroed where used (kFull: k % 1024 == 0)
  using Raw = f16x8[2];
  auto load_raw = [&](int64_t row, int p, Raw& h) {
    const _Float16* xr = x + row * k;
    const int c0 = p * kQuantCols + lane * 16;
    h[0] = *reinterpret_cast<const f16x8*>(xr + (kFull || c0 < k ? c0 : 0));
    h[1] = *reinterpret_cast<const f16x8*>(xr + (kFull || c0 + 8 < k ? c0 + 8 : 0));
  };
  // this lane's 16 values of pass p, rotated (unscaled) when kRotate; zeros past k
  auto rotate = [&](int p, const Raw& h, float (&v)[16]) {
    const int c0 = p * kQuantCols + lane * 16;
    const bool ok0 = kFull || c0 < k, ok1 = kFull || c0 + 8 < k;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[e] = ok0 ? static_cast<float>(h[0][e]) : 0.0f;
      v[e + 8] = ok1 ? static_cast<float>(h[1][e]) : 0.0f;
    }
    if constexpr (kRotate) {
      if (kFull || c0 < k) {
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
          const float4 t = *reinterpret_cast<const float4*>(mult + c0 + 4 * e4);
          v[4 * e4 + 0] *= t.x;
          v[4 * e4 + 1] *= t.y;
          v[4 * e4 + 2] *= t.z;
          v[4 * e4 + 3] *= t.w;
        }
      }
      // position bits 0..3 (in registers)
#pragma unroll
      for (int d = 1; d < 16; d <<= 1) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          if (e & d) continue;
          const float lo = v[e], hi = v[e + d];
          v[e] = lo + hi;
          v[e + d] = lo - hi;
        }
      }
      // position bit 4 (lane bit 0): lower lane L + H, upper lane L - H = L + (-H)
#pragma unroll
      for (int e = 0; e < 16; ++e) v[e] = dpp_xor1(v[e]) + v[e] * up1;
      // position bit 5 (lane bit 1)
#pragma unroll
      for (int e = 0; e < 16; ++e) v[e] = dpp_xor2(v[e]) + v[e] * up2;
    }
  };
  // quantise and store pass p
  auto store_pass = [&](int8_t* qr, int p, float (&v)[16], float t, float r, bool fast) {
    if (fast) {
#pragma unroll
      for (int e = 0; e < 16; ++e) v[e] = quant_div(v[e], t, r);
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) v[e] = v[e] / t;
    }
    const int c0 = p * kQuantCols + lane * 16;
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = quant_pack4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
    if (c0 + 8 < k) *reinterpret_cast<uint4*>(qr + c0) = make_uint4(w[0], w[1], w[2], w[3]);
    else if (c0 < k) *reinterpret_cast<uint2*>(qr + c0) = make_uint2(w[0], w[1]);
  };
  // the row's scale (written out) and the divisor of its values
  auto finish_scale = [&](int64_t row, float maximum, float& t, float& r, bool& fast) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) maximum = fmaxf(maximum, __shfl_xor(maximum, d, 64));
    float s;
    const QuantDivisor dv = quant_divisor<kRotate>(maximum, s);
    if (lane == 0) scale[row] = s;
    t = dv.t;
    r = dv.r;
    fast = dv.fast;
  };

  if constexpr (kHold) {
    // rows alternate between two register buffers: while one row is computed, the
    // next one's loads are in flight
    auto process = [&](int64_t row, Raw (&cur)[NP]) {
      float v[NP][16];
      float maximum = 0.0f;
      // columns past k hold zeros (whole 64-column blocks when rotating), which leave
      // the maximum of absolute values unchanged
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        rotate(p, cur[p], v[p]);
#pragma unroll
        for (int e = 0; e < 16; ++e) maximum = fmaxf(maximum, fabsf(v[p][e]));
      }
      float t, r;
      bool fast;
      finish_scale(row, maximum, t, r, fast);
      int8_t* qr = q + row * k;
#pragma unroll
      for (int p = 0; p < NP; ++p) store_pass(qr, p, v[p], t, r, fast);
    };
    auto load_row = [&](int64_t row, Raw (&buf)[NP]) {  // rows past m load row m - 1
      const int64_t rr = row < m ? row : m - 1;
#pragma unroll
      for (int p = 0; p < NP; ++p) load_raw(rr, p, buf[p]);
    };
    if constexpr (kPrefetch) {
      Raw a[NP], b[NP];
      load_row(first, a);
      for (int64_t row = first; row < m; row += 2 * stride) {
        load_row(row + stride, b);
        process(row, a);
        if (row + stride >= m) break;
        load_row(row + 2 * stride, a);
        process(row + stride, b);
      }
    } else {
      for (int64_t row = first; row < m; row += stride) {
        Raw a[NP];
        load_row(row, a);
        process(row, a);
      }
    }
  } else {
    // wide rows: a first pass for the maximum, a second that recomputes and stores
    for (int64_t row = first; row < m; row += stride) {
      float maximum = 0.0f;
#pragma unroll 1
      for (int p = 0; p < NP; ++p) {
        Raw h;
        float v[16];
        load_raw(row, p, h);
        rotate(p, h, v);
#pragma unroll
        for (int e = 0; e < 16; ++e) maximum = fmaxf(maximum, fabsf(v[e]));
      }
      float t, r;
      bool fast;
      finish_scale(row, maximum, t, r, fast);
      int8_t* qr = q + row * k;
#pragma unroll 1
      for (int p = 0; p < NP; ++p) {
        Raw h;
        float v[16];
        load_raw(row, p, h);
        rotate(p, h, v);
        store_pass(qr, p, v, t, r, fast);
      }
    }
  }
}

// -------------------------------------------------------------------- GEMM --
// out[m, n] = fp16(((float)acc[m, n] * sa[m]) * sw[n] + (float)bias[n]) with the exact
// int32 acc[m, n] = sum_k q[m, k] * w[n, k].
//
// Workgroup tile: 256 tokens x 256 channels, 4 waves, each owning 128 channels x 128
// tokens as 4 x 4 blocks of v_mfma_i32_32x32x32_i8 with the weights as the first operand
// (a lane's accumulators then hold four consecutive channels of one token). K advances
// in 64-byte stages through a 4-deep LDS ring filled by direct-to-LDS 16-byte loads
// issued three stages ahead. Rows are 64 bytes with chunk c of row r stored at
// c ^ ((r >> 2) & 3): a wave's 16-byte fragment reads (32 consecutive rows, two chunks)
// then run without LDS bank conflicts (measured: 4 LDS cycles per read, against 8 with
// the chunk rotated by (r >> 1) ^ (r >> 3) and 16 with no rotation). One barrier per stage, between the two K-groups of the
// stage: before it the wave multiplies K-group 0 while its K-group 1 fragments load;
// after it, it issues the loads three stages ahead (into the buffer every wave has
// finished reading) and reads the next stage's K-group 0 while K-group 1 multiplies.
constexpr int kGemmBM = 256, kGemmBN = 256, kGemmRing = 4;
constexpr int kGemmStageA = kGemmBM * 64, kGemmStage = kGemmStageA + kGemmBN * 64;
constexpr int kGemmLoads = 8;  // direct-to-LDS loads per wave per stage

__device__ __attribute__((aligned(16))) const uint32_t g_zero_chunk[4] = {0u, 0u, 0u, 0u};

__device__ __forceinline__ int lds_off64(int row, int chunk) {
  return row * 64 + ((chunk ^ ((row >> 2) & 3)) << 4);
}

template <bool kDump, bool kTail>
__global__ __launch_bounds__(256, 1) void w8a8_gemm_kernel(const int8_t* __restrict__ qa, const float* __restrict__ sa,
                                                           const int8_t* __restrict__ w, const float* __restrict__ sw,
                                                           const _Float16* __restrict__ bias, int64_t m, int n, int k,
                                                           _Float16* __restrict__ out, int32_t* __restrict__ acc_out,
                                                           int ntiles) {
#pragma clang fp contract(off)
  constexpr int BM = kGemmBM, BN = kGemmBN, NS = kGemmRing;
  constexpr int RING = NS * kGemmStage;
  constexpr int EPI = BM * BN * 2;
  static_assert(EPI <= RING, "the epilogue tile reuses the ring");
  __shared__ __attribute__((aligned(16))) char smem[RING + (BM + BN) * 4 + BN * 2];
  float* const s_sa = reinterpret_cast<float*>(smem + RING);
  float* const s_sw = s_sa + BM;
  _Float16* const s_bias = reinterpret_cast<_Float16*>(s_sw + BN);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave >> 1, wm = wave & 1;
  // channel tiles innermost: the workgroups an XCD runs together share their token rows
  const int64_t item = xcd_remap(blockIdx.x, static_cast<int64_t>(gridDim.x));
  const int64_t mt = item / ntiles;
  const int nt = static_cast<int>(item - mt * ntiles);
  const int64_t m0 = mt * BM;
  const int n0 = nt * BN;

  for (int i = tid; i < BM; i += 256) s_sa[i] = m0 + i < m ? sa[m0 + i] : 0.0f;
  for (int j = tid; j < BN; j += 256) {
    const bool ok = n0 + j < n;
    s_sw[j] = ok ? sw[n0 + j] : 0.0f;
    s_bias[j] = (ok && bias != nullptr) ? bias[n0 + j] : static_cast<_Float16>(0.0f);
  }

  // load j (0..3) of this wave covers ring rows (4j + wave) * 16 .. +15; lane l fills row
  // + l / 4 at physical chunk l % 4, i.e. logical chunk (l % 4) ^ swizzle(row). Rows past
  // the matrix edge re-read the last row (their results are never stored). Sources are
  // a workgroup-uniform tile base plus a 32-bit per-lane offset (row * k + chunk), so
  // without a K tail (kTail false: k % 64 == 0) a load needs no per-lane arithmetic.
  const int S = (k + 63) >> 6;
  const int8_t* const a_tile = qa + m0 * k;
  const int8_t* const b_tile = w + static_cast<int64_t>(n0) * k;
  uint32_t aoff[4], boff[4];
  int coff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = (4 * j + wave) * 16 + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 2) & 3);
    coff[j] = c * 16;
    const int ar = m0 + r < m ? r : static_cast<int>(m - 1 - m0);
    const int br = n0 + r < n ? r : n - 1 - n0;
    aoff[j] = static_cast<uint32_t>(ar) * static_cast<uint32_t>(k) + coff[j];
    boff[j] = static_cast<uint32_t>(br) * static_cast<uint32_t>(k) + coff[j];
  }
  auto issue_one = [&](int s, int j) {  // load j of stage s: 0..3 tokens, 4..7 channels
    char* base = smem + (s % NS) * kGemmStage + (j < 4 ? 0 : kGemmStageA) + (4 * (j & 3) + wave) * 1024;
    const int kb = s * 64;
    const int8_t* src = (j < 4 ? a_tile : b_tile) + kb + (j < 4 ? aoff[j & 3] : boff[j & 3]);
    if (kTail) {
      const bool ok = kb + coff[j & 3] < k;
      lds_dma16(ok ? static_cast<const void*>(src) : static_cast<const void*>(g_zero_chunk), base);
    } else {
      lds_dma16(src, base);
    }
  };
  auto issue = [&](int s) {
#pragma unroll
    for (int j = 0; j < kGemmLoads; ++j) issue_one(s, j);
  };

  i32x16 acc[4][4];  // [channel block][token block]
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[nb][mb][v] = 0;
  u32x4 fw[2][4], fq[2][4];  // fragments of K-group 0 / 1
  // fragment read i of K-group G of stage s: 0..3 channel blocks, 4..7 token blocks
  auto frag_one = [&](int s, auto gc, int i) {
    constexpr int G = decltype(gc)::value;
    const char* A = smem + (s % NS) * kGemmStage;
    const int c = 2 * G + (lane >> 5);
    if (i < 4)
      fw[G][i] = *reinterpret_cast<const u32x4*>(A + kGemmStageA + lds_off64(wn * 128 + i * 32 + (lane & 31), c));
    else
      fq[G][i - 4] = *reinterpret_cast<const u32x4*>(A + lds_off64(wm * 128 + (i - 4) * 32 + (lane & 31), c));
  };
  auto frags = [&](int s, auto gc) {
#pragma unroll
    for (int i = 0; i < 8; ++i) frag_one(s, gc, i);
  };
  // MFMA i of K-group G: channel block i / 4, token block i % 4
  auto mma_one = [&](auto gc, int i) {
    constexpr int G = decltype(gc)::value;
    acc[i >> 2][i & 3] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, fw[G][i >> 2]),
                                                             __builtin_bit_cast(i32x4, fq[G][i & 3]), acc[i >> 2][i & 3],
                                                             0, 0, 0);
  };
  auto mma = [&](auto gc) {
#pragma unroll
    for (int i = 0; i < 16; ++i) mma_one(gc, i);
  };
  using G0 = std::integral_constant<int, 0>;
  using G1 = std::integral_constant<int, 1>;

  // Loads of stage s + 3 are spread over two half-stages to keep the vector memory path
  // busy without bursts: channel rows (loads 4..7) during the second half of stage s,
  // token rows (loads 0..3) during the first half of stage s + 1. Either way every wave
  // has passed the barrier of stage s, so the buffer of stage s - 1 is free.
  //
  // First half of stage s: K-group 0 MFMAs; after each of the first eight one K-group 1
  // fragment read, after every other one of the last eight (with `dma`) one token-row
  // load of stage s + 2.
  auto half0 = [&](int s, bool dma) {
    wait_lgkm0();  // K-group 0 fragments (read during the previous K-group 1 MFMAs) are in
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      mma_one(G0{}, i);
      __builtin_amdgcn_sched_barrier(0);
      if (i < 8) {
        frag_one(s, G1{}, i);
      } else if (dma && (i & 1)) {
        issue_one(s + NS - 2, (i - 8) >> 1);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Second half: K-group 1 MFMAs; after each of the first eight one K-group 0 fragment
  // read of stage s + 1, after every other one of the last eight (with `dma`) one
  // channel-row load of stage s + 3.
  auto half1 = [&](int s, bool dma) {
    wait_lgkm0();  // K-group 1 fragments (read during the K-group 0 MFMAs) are in
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      mma_one(G1{}, i);
      __builtin_amdgcn_sched_barrier(0);
      if (i < 8) {
        frag_one(s + 1, G0{}, i);
      } else if (dma && (i & 1)) {
        issue_one(s + NS - 1, 4 + ((i - 8) >> 1));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Barrier of stage s: this wave's part of stage s + 1 has landed (loads issued later:
  // stage s + 2, i.e. kGemmLoads of them while it exists) and every wave is done reading
  // stage s - 1.
  auto sync = [&](int s) {
    if (s + 2 < S) wait_vmcnt<kGemmLoads>();
    else wait_vmcnt<0>();
    raw_barrier();
  };

  // prologue: stages 0..2 in full
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < S) issue(s);
  if (S > 2) wait_vmcnt<2 * kGemmLoads>();
  else if (S > 1) wait_vmcnt<kGemmLoads>();
  else wait_vmcnt<0>();
  raw_barrier();
  frags(0, G0{});
  int s = 0;
  if (S > 1) {  // stage 0: its first half has no token rows to load (stage 2 is loaded)
    half0(0, false);
    sync(0);
    half1(0, NS - 1 < S);
    s = 1;
  }
  for (; s + NS - 1 < S; ++s) {  // steady state: both halves load
    half0(s, true);
    sync(s);
    half1(s, true);
  }
  if (s + NS - 2 < S && s + 1 < S) {  // token rows of the last stage remain
    half0(s, true);
    sync(s);
    half1(s, false);
    ++s;
  }
  for (; s + 1 < S; ++s) {  // nothing left to load
    half0(s, false);
    sync(s);
    half1(s, false);
  }
  if (S > 0) {  // the final stage
    wait_lgkm0();
    frags(S - 1, G1{});
    mma(G0{});
    mma(G1{});
  }

  // epilogue: channels wn*128 + nb*32 + 8*(v/4) + 4*(l/32) + v%4, token wm*128 + mb*32 + l%32
  if (kDump) {
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const int64_t row = m0 + wm * 128 + mb * 32 + (lane & 31);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int col = n0 + wn * 128 + nb * 32 + 8 * q + 4 * (lane >> 5);
          if (row >= m) continue;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (col + e < n) acc_out[row * n + col + e] = acc[nb][mb][4 * q + e];
        }
      }
  }
  wait_vmcnt<0>();
  __syncthreads();  // every wave is done with the ring: it becomes the output tile
  _Float16* C = reinterpret_cast<_Float16*>(smem);
  constexpr int CROW = BN * 2;  // bytes per output row in LDS; 16-byte chunks swizzled by row
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    const int i = wm * 128 + mb * 32 + (lane & 31);
    const float sar = s_sa[i];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int j0 = wn * 128 + nb * 32 + 8 * q + 4 * (lane >> 5);
        _Float16 h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float prod = static_cast<float>(acc[nb][mb][4 * q + e]) * sar;
          h[e] = static_cast<_Float16>(prod * s_sw[j0 + e] + static_cast<float>(s_bias[j0 + e]));
        }
        const int chunk = (j0 >> 3) ^ (i & 31);
        *reinterpret_cast<uint2*>(reinterpret_cast<char*>(C) + i * CROW + chunk * 16 + (j0 & 4) * 2) =
            __builtin_bit_cast(uint2, h);
      }
    }
  }
  __syncthreads();
  constexpr int CPR = BN / 8;  // 16-byte chunks per row
  const bool vec = (n & 7) == 0;
  for (int q = tid; q < BM * CPR; q += 256) {
    const int i = q / CPR, cc = q % CPR;
    const int64_t row = m0 + i;
    const int col = n0 + cc * 8;
    if (row >= m || col >= n) continue;
    const u32x4 v = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(C) + i * CROW + ((cc ^ (i & 31)) * 16));
    if (vec) {
      *reinterpret_cast<u32x4*>(out + row * n + col) = v;
    } else {
      const _Float16* pv = reinterpret_cast<const _Float16*>(&v);
      for (int e = 0; e < 8 && col + e < n; ++e) out[row * n + col + e] = pv[e];
    }
  }
}

// Persistent variant for full tiles (m, n >= 256, n % 8 == 0, k % 64 == 0, k >= 256): one
// workgroup per CU walks a list of tiles while the stage pipeline above runs on without a
// break: the next tile's first stages load during the current tile's last ones, and the
// per-tile work around the K loop shrinks to the epilogue.
//  * Tiles: the last tile of each dimension is moved back to end at m (n), so every tile
//    is full and in bounds; where tiles overlap, both compute and store the same bits.
//  * Work list: the chip deals workgroups round-robin over its 8 XCDs; each XCD's
//    workgroups take a contiguous range of tiles (channel tiles innermost), so the tiles
//    an XCD runs together share their token rows in its L2.
//  * Scales: sa / sw / bias of a tile arrive by three 4-byte direct-to-LDS loads per wave
//    at the tile's first stage, into one of two LDS slots.
//  * Epilogue: after the last MFMAs of a tile, the ring buffer of that stage (free: every
//    wave is past its reads) stages the int32 accumulators in eight 32-token chunks,
//    written straight from the accumulator registers by the two waves holding those
//    tokens; every thread then converts one fixed 8-channel group of 4 rows per chunk
//    (dequant + bias, fp16) and stores it as one 16-byte row chunk. The stores drain while
//    the next tile computes.
//  * Counting: every wave issues the same number of vector memory operations (no
//    predicated loads or stores), so the vmcnt waits are exact: at the barrier of stage g
//    the operations issued after stage g + 1's last load are stage g + 2's loads (8) and,
//    at a tile's first stage, the previous tile's 32 stores and this tile's 3 scale loads.
constexpr int kGemmScale = kGemmBM * 4 + kGemmBN * 4 + kGemmBN * 2;  // sa, sw, bias of one tile
constexpr int kGemmStores = 32;                                       // epilogue stores per wave
constexpr int kGemmScaleLoads = 3;                                    // scale loads per wave per tile

__device__ __attribute__((aligned(16))) const uint32_t g_zero_bias[kGemmBN / 2] = {};

__device__ __forceinline__ void lds_dma4(const void* src, char* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(lds_wave_base), 4, 0, 0);
}

// kDump: the read-back threads also store the int32 accumulators they convert (the
// bit-exact gate of this kernel's K loop and tile walk) and drain every store at the end
// of each epilogue, so the waits counted for the fused-output form stay conservative.
template <bool kDump>
__global__ __launch_bounds__(256, 1) void w8a8_gemm_persistent_kernel(
    const int8_t* __restrict__ qa, const float* __restrict__ sa, const int8_t* __restrict__ w,
    const float* __restrict__ sw, const _Float16* __restrict__ bias, int64_t m, int n, int k,
    _Float16* __restrict__ out, int32_t* __restrict__ acc_out, int ntiles_n, int64_t total) {
#pragma clang fp contract(off)
  constexpr int NS = kGemmRing;
  constexpr int RING = NS * kGemmStage;
  __shared__ __attribute__((aligned(16))) char smem[RING + 2 * kGemmScale];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave >> 1, wm = wave & 1;

  // this workgroup's tiles: lo + L + i * P_x within the XCD's range [lo, hi)
  const int P = static_cast<int>(gridDim.x);
  const int x = static_cast<int>(blockIdx.x) & 7, L = static_cast<int>(blockIdx.x) >> 3;
  const int Px = P / 8 + (x < P % 8 ? 1 : 0);
  const int64_t per = total / 8, rem = total % 8;
  const int64_t lo = x * per + (x < rem ? x : rem);
  const int64_t hi = lo + per + (x < rem ? 1 : 0);
  const int64_t mine = hi - lo > L ? (hi - lo - L + Px - 1) / Px : 0;
  const int S = k >> 6;
  const int64_t G = mine * S;
  if (G == 0) return;
  auto origin = [&](int64_t t, int64_t& m0, int& n0) {
    const int64_t item = lo + L + t * Px;
    const int64_t mt = item / ntiles_n;
    const int nt = static_cast<int>(item - mt * ntiles_n);
    m0 = mt * kGemmBM < m - kGemmBM ? mt * kGemmBM : m - kGemmBM;
    n0 = nt * kGemmBN < n - kGemmBN ? nt * kGemmBN : n - kGemmBN;
  };

  // per-lane source offsets inside a tile (see the non-persistent kernel for the layout)
  uint32_t roff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = (4 * j + wave) * 16 + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 2) & 3);
    roff[j] = static_cast<uint32_t>(r) * static_cast<uint32_t>(k) + c * 16;
  }
  // load cursors: the next stage whose token (A) / channel (B) rows are to be issued
  struct Cursor {
    int64_t t;
    int s, slot;
    const int8_t* base;  // tile rows + 64 s
  };
  auto cursor_at_tile = [&](Cursor& c, bool tokens) {
    int64_t m0;
    int n0;
    origin(c.t, m0, n0);
    c.base = tokens ? qa + m0 * k : w + static_cast<int64_t>(n0) * k;
  };
  auto advance = [&](Cursor& c, bool tokens) {
    c.slot = (c.slot + 1) & (NS - 1);
    if (++c.s == S) {
      c.s = 0;
      ++c.t;
      if (c.t < mine) cursor_at_tile(c, tokens);
    } else {
      c.base += 64;
    }
  };
  Cursor ct{0, 0, 0, nullptr}, cc{0, 0, 0, nullptr};
  cursor_at_tile(ct, true);
  cursor_at_tile(cc, false);
  auto issue_tokens = [&](int j) {  // load j (0..3) of the token cursor's stage
    lds_dma16(ct.base + roff[j], smem + ct.slot * kGemmStage + (4 * j + wave) * 1024);
  };
  auto issue_channels = [&](int j) {
    lds_dma16(cc.base + roff[j], smem + cc.slot * kGemmStage + kGemmStageA + (4 * j + wave) * 1024);
  };
  auto issue_scales = [&](int64_t t) {
    int64_t m0;
    int n0;
    origin(t, m0, n0);
    char* region = smem + RING + (t & 1) * kGemmScale;
    lds_dma4(sa + m0 + wave * 64 + lane, region + wave * 256);
    lds_dma4(sw + n0 + wave * 64 + lane, region + kGemmBM * 4 + wave * 256);
    const uint32_t* b = bias != nullptr ? reinterpret_cast<const uint32_t*>(bias + n0) : g_zero_bias;
    lds_dma4(b + (wave & 1) * 64 + lane, region + (kGemmBM + kGemmBN) * 4 + (wave & 1) * 256);
  };

  i32x16 acc[4][4];
  u32x4 fw[2][4], fq[2][4];
  auto frag_one = [&](int slot, auto gc, int i) {
    constexpr int Gk = decltype(gc)::value;
    const char* A = smem + slot * kGemmStage;
    const int c = 2 * Gk + (lane >> 5);
    if (i < 4)
      fw[Gk][i] = *reinterpret_cast<const u32x4*>(A + kGemmStageA + lds_off64(wn * 128 + i * 32 + (lane & 31), c));
    else
      fq[Gk][i - 4] = *reinterpret_cast<const u32x4*>(A + lds_off64(wm * 128 + (i - 4) * 32 + (lane & 31), c));
  };
  const i32x16 zero16 = {};
  auto mma_one = [&](auto gc, int i, auto fc) {  // fc: first K-group of a tile (zero accumulators)
    constexpr int Gk = decltype(gc)::value;
    constexpr bool kFirst = decltype(fc)::value;
    acc[i >> 2][i & 3] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, fw[Gk][i >> 2]),
                                                             __builtin_bit_cast(i32x4, fq[Gk][i & 3]),
                                                             kFirst ? zero16 : acc[i >> 2][i & 3], 0, 0, 0);
  };
  using G0 = std::integral_constant<int, 0>;
  using G1 = std::integral_constant<int, 1>;

  // prologue: tile 0's scales, then stages 0..2 in full
  issue_scales(0);
#pragma unroll
  for (int st = 0; st < NS - 1; ++st) {
#pragma unroll
    for (int j = 0; j < 4; ++j) issue_tokens(j);
#pragma unroll
    for (int j = 0; j < 4; ++j) issue_channels(j);
    advance(ct, true);
    advance(cc, false);
  }
  wait_vmcnt<2 * kGemmLoads>();  // G >= S >= 4: stages 1 and 2 may stay in flight
  raw_barrier();
#pragma unroll
  for (int i = 0; i < 8; ++i) frag_one(0, G0{}, i);

  int s = 0;  // stage of the current tile
  int64_t t = 0;
  // Stage g of the stream. MODE 0: g = 0 (its token rows were part of the prologue);
  // 1: steady (token rows of stage g + 2, channel rows of stage g + 3); 2: g = G - 3
  // (token rows only); 3: g = G - 2 (no loads); 4: g = G - 1 (nothing follows). `first`
  // marks a tile's first stage: zero accumulators, the tile's scales, and the previous
  // tile's epilogue stores still in flight at the barrier.
  auto stage = [&](int64_t g, auto modec) {
    constexpr int MODE = decltype(modec)::value;
    constexpr bool tok = MODE == 1 || MODE == 2, chn = MODE <= 1, nxt = MODE != 4;
    const int slot = static_cast<int>(g & (NS - 1));
    const bool first = s == 0;
    // first half: K-group 0 MFMAs (zero accumulators at a tile's first stage), K-group 1
    // fragment reads, token-row loads of stage g + 2 and, at a tile's first stage, its scales
    wait_lgkm0();
    if (first && g > 0) issue_scales(t);
    __builtin_amdgcn_sched_barrier(0);
    auto half0 = [&](auto fc) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        mma_one(G0{}, i, fc);
        __builtin_amdgcn_sched_barrier(0);
        if (i < 8) {
          frag_one(slot, G1{}, i);
        } else if constexpr (tok) {
          if (i & 1) issue_tokens((i - 8) >> 1);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    if (first) half0(std::true_type{});
    else half0(std::false_type{});
    if constexpr (tok) advance(ct, true);
    if constexpr (MODE == 3) {
      wait_vmcnt<0>();
      raw_barrier();
    } else if constexpr (nxt) {
      if (first && g > 0) wait_vmcnt<kGemmLoads + kGemmStores + kGemmScaleLoads>();
      else wait_vmcnt<kGemmLoads>();
      raw_barrier();
    }
    // second half: K-group 1 MFMAs, K-group 0 fragment reads of stage g + 1, channel-row
    // loads of stage g + 3
    wait_lgkm0();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      mma_one(G1{}, i, std::false_type{});
      __builtin_amdgcn_sched_barrier(0);
      if (i < 8) {
        if constexpr (nxt) frag_one((slot + 1) & (NS - 1), G0{}, i);
      } else if constexpr (chn) {
        if (i & 1) issue_channels((i - 8) >> 1);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (chn) advance(cc, false);

    if (++s == S) {  // epilogue of tile t
      s = 0;
      if constexpr (!nxt) raw_barrier();  // the final stage has no barrier of its own
      int64_t m0;
      int n0;
      origin(t, m0, n0);
      const char* region = smem + RING + (t & 1) * kGemmScale;
      const float* s_sa = reinterpret_cast<const float*>(region);
      const float* s_sw = s_sa + kGemmBM;
      const _Float16* s_bias = reinterpret_cast<const _Float16*>(s_sw + kGemmBN);
      char* stg = smem + slot * kGemmStage;
      // read-back role: this thread converts channels cb .. cb + 7 of rows tid / 32 + 8 i
      const int grp = tid & 31, cb = grp * 8;
      const f32x4 sw0 = *reinterpret_cast<const f32x4*>(s_sw + cb);
      const f32x4 sw1 = *reinterpret_cast<const f32x4*>(s_sw + cb + 4);
      const f16x8 bv = *reinterpret_cast<const f16x8*>(s_bias + cb);
#pragma unroll
      for (int c = 0; c < 8; ++c) {  // tokens 32 c .. 32 c + 31 = block mb = c % 4 of the waves with wm = c / 4
        if (wm == (c >> 2)) {
          const int row = lane & 31;
#pragma unroll
          for (int nb = 0; nb < 4; ++nb)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int ch = wn * 32 + nb * 8 + 2 * q + (lane >> 5);  // 4-channel group
              const i32x4 v = {acc[nb][c & 3][4 * q], acc[nb][c & 3][4 * q + 1], acc[nb][c & 3][4 * q + 2],
                               acc[nb][c & 3][4 * q + 3]};
              *reinterpret_cast<i32x4*>(stg + row * 1024 + ((ch ^ row) << 4)) = v;
            }
        }
        wait_lgkm0();
        raw_barrier();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = (tid >> 5) + 8 * i;
          const float sar = s_sa[c * 32 + row];
          const i32x4 lo = *reinterpret_cast<const i32x4*>(stg + row * 1024 + (((2 * grp) ^ row) << 4));
          const i32x4 hi = *reinterpret_cast<const i32x4*>(stg + row * 1024 + (((2 * grp + 1) ^ row) << 4));
          f16x8 y;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            y[e] = static_cast<_Float16>((static_cast<float>(lo[e]) * sar) * sw0[e] + static_cast<float>(bv[e]));
            y[e + 4] = static_cast<_Float16>((static_cast<float>(hi[e]) * sar) * sw1[e] + static_cast<float>(bv[e + 4]));
          }
          *reinterpret_cast<f16x8*>(out + (m0 + 32 * c + row) * n + n0 + cb) = y;
          if constexpr (kDump) {
            int32_t* const dst = acc_out + (m0 + 32 * c + row) * n + n0 + cb;
            *reinterpret_cast<i32x4*>(dst) = lo;
            *reinterpret_cast<i32x4*>(dst + 4) = hi;
          }
        }
        wait_lgkm0();
        raw_barrier();
      }
      if constexpr (kDump) wait_vmcnt<0>();
      ++t;
    }
  };
  using M0 = std::integral_constant<int, 0>;
  using M1 = std::integral_constant<int, 1>;
  using M2 = std::integral_constant<int, 2>;
  using M3 = std::integral_constant<int, 3>;
  using M4 = std::integral_constant<int, 4>;
  stage(0, M0{});
  for (int64_t g = 1; g + 3 < G; ++g) stage(g, M1{});
  stage(G - 3, M2{});
  stage(G - 2, M3{});
  stage(G - 1, M4{});
}

// ---------------------------------------------------------- ping-pong GEMM --
// 256 x 256 tiles, 8 waves in two groups of four. Group g holds tokens 128 g .. +127;
// wave q of a group holds channels 64 q .. +63 (2 x 4 blocks of v_mfma_i32_32x32x32_i8,
// 128 accumulator registers), so two waves share each SIMD. The groups alternate: in
// phase A of stage s group 0 multiplies stage s while group 1 issues its share of the
// loads of stage s + 3 and reads its fragments of stage s; in phase B group 1 multiplies
// while group 0 issues its loads and reads its fragments of stage s + 1. One barrier
// ends each phase, so each SIMD always has one wave with a full phase of MFMAs (16, 512
// cycles) queued while the other one feeds LDS: loads and matrix work overlap by
// construction instead of by the interleaving of one wave's instruction stream.
//  * Ring: 4 stages of 64 bytes of K (256 token rows + 256 channel rows, 32 KB), rows in
//    the 64-byte rotated layout (chunk c of row r at c ^ ((r >> 2) & 3)). Each wave loads
//    16 rows of tokens and 16 rows of channels per 8 KB half (4 direct-to-LDS loads per
//    stage); a stage's loads are issued three stages ahead (group 1 in phase A, group 0
//    in phase B of stage s - 3) into the slot of stage s - 1, which both groups finished
//    reading before the barrier that opens phase A(s).
//  * Waits: before the barrier that ends phase A(s), each wave waits for its loads of
//    stage s + 1 (group 1 has the loads of s + 2 and s + 3 behind them, group 0 those of
//    s + 2), so stage s + 1 is complete when group 0 reads it in phase B(s).
//  * Epilogue: each wave converts its accumulators in registers (the reference's
//    fp16(((float)acc * sa) * sw + bias), no contraction) into an fp16 tile in LDS, then
//    every thread stores whole 16-byte row chunks (512-byte rows, coalesced).
//  * Tile order: the chip deals workgroups round-robin over its 8 XCDs; XCD x takes
//    channel-tile group x % G and token part x / G, channel tiles innermost, so the
//    channel rows of its group stay in its L2 and the tiles sharing a token block run
//    together (G chosen on the host from the operand sizes).
constexpr int kPPStage = 32768, kPPHalf = 16384, kPPRing = 4;
constexpr int kRawBufferFlags = 0x00020000;  // buffer descriptor word 3 for raw byte loads

__device__ __forceinline__ __attribute__((address_space(3))) void* lds_ptr(char* p) {
  return (__attribute__((address_space(3))) void*)(p);
}

// 32-bit LDS address of a pointer into shared memory (for LDS instructions in asm)
__device__ __forceinline__ uint32_t lds_addr(char* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds_ptr(p)));
}

template <bool kDump>
__global__ __launch_bounds__(512, 1) void w8a8_gemm_pp_kernel(const int8_t* __restrict__ qa, const float* __restrict__ sa,
                                                              const int8_t* __restrict__ w, const float* __restrict__ sw,
                                                              const _Float16* __restrict__ bias, int64_t m, int n, int k,
                                                              _Float16* __restrict__ out, int32_t* __restrict__ acc_out,
                                                              int64_t mt_count, int nt_count, int groups) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) char smem[kPPRing * kPPStage + 256 * 4 * 2 + 256 * 2];
  float* const s_sa = reinterpret_cast<float*>(smem + kPPRing * kPPStage);
  float* const s_sw = s_sa + 256;
  _Float16* const s_bias = reinterpret_cast<_Float16*>(s_sw + 256);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = wave >> 2, q = wave & 3;

  // this block's tile
  const int xcd = static_cast<int>(blockIdx.x & 7);
  const int64_t local = blockIdx.x >> 3;
  const int parts = 8 / groups;
  const int cg = xcd % groups, part = xcd / groups;
  const int cpg = (nt_count + groups - 1) / groups;
  const int64_t mpp = (mt_count + parts - 1) / parts;
  const int nt_lo = cg * cpg, nt_hi = nt_count < nt_lo + cpg ? nt_count : nt_lo + cpg;
  const int ntg = nt_hi - nt_lo;
  const int64_t mt_lo = part * mpp, mt_hi = mt_count < mt_lo + mpp ? mt_count : mt_lo + mpp;
  if (ntg <= 0) return;
  const int64_t mt = mt_lo + local / ntg;
  if (mt >= mt_hi) return;
  const int64_t m0 = mt * 256;
  const int n0 = (nt_lo + static_cast<int>(local % ntg)) * 256;

  // scales and bias of the tile (older than every ring load, so complete at the first wait)
  {
    const int64_t ra = m0 + (wave & 3) * 64 + lane;
    const int cb = n0 + (wave & 3) * 64 + lane;
    if (wave < 4) lds_dma4(sa + (ra < m ? ra : m - 1), reinterpret_cast<char*>(s_sa) + (wave & 3) * 256);
    else lds_dma4(sw + (cb < n ? cb : n - 1), reinterpret_cast<char*>(s_sw) + (wave & 3) * 256);
    if (wave < 2) {
      const int d = n0 / 2 + wave * 64 + lane;  // bias dword: channels 2 d, 2 d + 1 (n is even)
      const uint32_t* b32 = bias != nullptr ? reinterpret_cast<const uint32_t*>(bias) + (d < n / 2 ? d : n / 2 - 1)
                                            : g_zero_bias + ((wave * 64 + lane) & 127);
      lds_dma4(b32, reinterpret_cast<char*>(s_bias) + wave * 256);
    }
  }

  // This wave's 4 loads per stage: token rows and channel rows 128 g + (2 q + j) * 16 +
  // lane / 4, through buffer descriptors of the tile's rows (rows past the matrix read
  // zeros), with the stage's K offset as the scalar offset: no vector arithmetic per load.
  const int rows_a = m - m0 < 256 ? static_cast<int>(m - m0) : 256;
  const int rows_b = n - n0 < 256 ? n - n0 : 256;
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(qa + m0 * k), 0, rows_a * k,
                                                                      kRawBufferFlags);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t*>(w + static_cast<int64_t>(n0) * k), 0, rows_b * k, kRawBufferFlags);
  const int c16 = ((lane & 3) ^ ((lane >> 4) & 3)) * 16;
  int vo[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) vo[j] = (128 * g + (2 * q + j) * 16 + (lane >> 2)) * k + c16;
  auto issue = [&](int s, auto slc) {
    constexpr int SL = decltype(slc)::value;
#pragma unroll
    for (int j = 0; j < 2; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, lds_ptr(smem + SL * kPPStage + (8 * g + 2 * q + j) * 1024), 16,
                                               vo[j], s * 64, 0, 0);
#pragma unroll
    for (int j = 0; j < 2; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, lds_ptr(smem + SL * kPPStage + kPPHalf + (8 * g + 2 * q + j) * 1024),
                                               16, vo[j], s * 64, 0, 0);
  };

  // fragment reads: per-lane bases for each K-group (slots 0-1 and 2-3, so that the
  // slot and block parts of every address are immediate offsets)
  u32x4 fw[2][2], fq[2][4];  // [K-group][channel block] / [K-group][token block]
  const char* bw[2][2];
  const char* bq[2][2];
#pragma unroll
  for (int G = 0; G < 2; ++G) {
    const int c = 2 * G + (lane >> 5);
    bw[G][0] = smem + kPPHalf + lds_off64(64 * q + (lane & 31), c);
    bq[G][0] = smem + lds_off64(128 * g + (lane & 31), c);
    bw[G][1] = bw[G][0] + 2 * kPPStage;
    bq[G][1] = bq[G][0] + 2 * kPPStage;
  }
  auto read_frags = [&](auto slc) {
    constexpr int SL = decltype(slc)::value;
#pragma unroll
    for (int G = 0; G < 2; ++G) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
        fw[G][nb] = *reinterpret_cast<const u32x4*>(bw[G][SL >> 1] + (SL & 1) * kPPStage + nb * 2048);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
        fq[G][mb] = *reinterpret_cast<const u32x4*>(bq[G][SL >> 1] + (SL & 1) * kPPStage + mb * 2048);
    }
  };
  i32x16 acc[2][4];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[nb][mb][v] = 0;
  auto compute = [&]() {
    wait_lgkm0();
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int G = 0; G < 2; ++G)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
          acc[nb][mb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, fw[G][nb]),
                                                            __builtin_bit_cast(i32x4, fq[G][mb]), acc[nb][mb], 0, 0, 0);
    __builtin_amdgcn_s_setprio(0);
  };
  auto wait_after = [&](int after) {
    if (after == 8) wait_vmcnt<8>();
    else if (after == 4) wait_vmcnt<4>();
    else wait_vmcnt<0>();
  };
  using SL0 = std::integral_constant<int, 0>;
  using SL1 = std::integral_constant<int, 1>;
  using SL2 = std::integral_constant<int, 2>;
  using SL3 = std::integral_constant<int, 3>;

  // Prologue: stages 0 and 1 from both groups, stage 2 from group 1 (group 0 issues its
  // share in phase -1, where it also reads the fragments of stage 0); stage 0 complete.
  const int S = k >> 6;  // a multiple of 4
  issue(0, SL0{});
  issue(1, SL1{});
  if (g == 1) {
    issue(2, SL2{});
    wait_vmcnt<8>();
  } else {
    wait_vmcnt<4>();
  }
  raw_barrier();
  if (g == 0) {
    issue(2, SL2{});
    read_frags(SL0{});
  }
  raw_barrier();

  // Stage s is two phases: A(s), group 0 multiplies while group 1 prepares (its loads of
  // stage s + 3, its fragments of stage s), and B(s), group 1 multiplies while group 0
  // prepares (loads of s + 3, fragments of s + 1). Each group runs its own straight-line
  // loop, four stages (one per ring slot) per iteration; both pass the same two barriers
  // per stage. Past the last stage the fragment reads read a stale slot nothing multiplies.
  auto g0_stage = [&](int s, auto slc) {
    constexpr int SL = decltype(slc)::value;
    __builtin_amdgcn_sched_barrier(0);
    compute();  // A(s)
    __builtin_amdgcn_sched_barrier(0);
    if (s + 1 < S) wait_after(s + 2 < S ? 4 : 0);  // own loads of stage s + 1 landed
    raw_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if (s + 3 < S) issue(s + 3, std::integral_constant<int, (SL + 3) & 3>{});  // B(s)
    read_frags(std::integral_constant<int, (SL + 1) & 3>{});
    __builtin_amdgcn_sched_barrier(0);
    raw_barrier();
  };
  auto g1_stage = [&](int s, auto slc) {
    constexpr int SL = decltype(slc)::value;
    __builtin_amdgcn_sched_barrier(0);
    if (s + 3 < S) issue(s + 3, std::integral_constant<int, (SL + 3) & 3>{});  // A(s)
    read_frags(slc);
    __builtin_amdgcn_sched_barrier(0);
    if (s + 1 < S) wait_after((s + 2 < S ? 4 : 0) + (s + 3 < S ? 4 : 0));
    raw_barrier();
    __builtin_amdgcn_sched_barrier(0);
    compute();  // B(s)
    __builtin_amdgcn_sched_barrier(0);
    raw_barrier();
  };
  if (g == 0) {
    for (int s = 0; s < S; s += 4) {
      g0_stage(s, SL0{});
      g0_stage(s + 1, SL1{});
      g0_stage(s + 2, SL2{});
      g0_stage(s + 3, SL3{});
    }
  } else {
    for (int s = 0; s < S; s += 4) {
      g1_stage(s, SL0{});
      g1_stage(s + 1, SL1{});
      g1_stage(s + 2, SL2{});
      g1_stage(s + 3, SL3{});
    }
  }

  // epilogue: the ring becomes a 256 x 256 fp16 tile (512-byte rows, 16-byte chunks
  // rotated by the row) written from the accumulators, then stored row-contiguously
  char* const C = smem;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    const int row = 128 * g + mb * 32 + (lane & 31);
    const float sar = s_sa[row];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int col = 64 * q + nb * 32 + 8 * q4 + 4 * (lane >> 5);
        const f32x4 swv = *reinterpret_cast<const f32x4*>(s_sw + col);
        _Float16 bv[4];
        __builtin_memcpy(bv, s_bias + col, sizeof(bv));
        _Float16 h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          h[e] = static_cast<_Float16>((static_cast<float>(acc[nb][mb][4 * q4 + e]) * sar) * swv[e] +
                                       static_cast<float>(bv[e]));
        *reinterpret_cast<uint2*>(C + row * 512 + (((col >> 3) ^ (row & 31)) << 4) + (col & 7) * 2) =
            __builtin_bit_cast(uint2, h);
        if constexpr (kDump) {
          if (m0 + row < m && n0 + col < n) {  // n % 8 == 0: the 4 channels are all inside
            const i32x4 v = {acc[nb][mb][4 * q4], acc[nb][mb][4 * q4 + 1], acc[nb][mb][4 * q4 + 2],
                             acc[nb][mb][4 * q4 + 3]};
            *reinterpret_cast<i32x4*>(acc_out + (m0 + row) * n + n0 + col) = v;
          }
        }
      }
    }
  }
  wait_lgkm0();
  raw_barrier();
#pragma unroll 4
  for (int i = 0; i < 16; ++i) {
    const int idx = i * 512 + tid;
    const int row = idx >> 5, ch = idx & 31;
    if (m0 + row < m && n0 + ch * 8 < n)
      *reinterpret_cast<u32x4*>(out + (m0 + row) * n + n0 + ch * 8) =
          *reinterpret_cast<const u32x4*>(C + row * 512 + ((ch ^ (row & 31)) << 4));
  }
}

// ------------------------------------------------ persistent ping-pong GEMM --
// The ping-pong kernel's stage loop, run persistently over a list of tiles per
// workgroup (the same XCD-aware order). The stage sequence continues across tiles: the
// loads of a tile's stages 0-2 are issued during the previous tile's last three stages,
// so no tile waits for its first loads.
//  * Epilogue, after a tile's last stage: its ring slot (3) is the only free one (the
//    next tile's stages 0-2 are in flight into slots 0-2). The tile leaves in four rounds
//    of 64 rows: each wave converts one 32-row block of its accumulators (the reference's
//    fp16(((float)acc * sa) * sw + bias), no contraction), writes it to slot 3 as fp16
//    (512-byte rows, 16-byte chunks rotated by the row), and after a barrier every thread
//    stores four 16-byte row chunks. These stores queue behind the next tile's first
//    loads and drain while it runs.
//  * Stores go through a buffer descriptor over the tile's valid rows, and a chunk past
//    the last channel gets an offset past the descriptor: no store is predicated, every
//    wave issues the same operations and the vmcnt waits are exact. At stages 0 and 1 of
//    a tile the operations younger than the awaited loads include the epilogue's 16
//    stores and the next tile's 2 scale loads.
//  * Scales: sa, sw and bias of the next tile are loaded (2 direct-to-LDS loads per wave,
//    sa and sw in one, bias halves in the other) right after the epilogue that last read
//    them; group 0 widens the bias to fp32 in phase B of stage 3, after every wave's scale
//    loads have passed a wait.
//  * A tile's first MFMAs take a zero accumulator operand (no clearing). After its last
//    tile a workgroup still issues the loads of a tile past its list through empty
//    descriptors (zeros into slots nobody reads), so the stage code has no tail form; it
//    waits for all of them before it exits.
constexpr int kPQScale = kPPRing * kPPStage;  // s_sa (1 KB), s_sw (1 KB), bias fp16 (512 B), bias fp32 (1 KB)
constexpr int kPQEpiOps = 16 + 2;              // epilogue stores + scale loads per wave
constexpr int kCachePolicyNT = 2;  // the NT bit of a buffer instruction's cache-policy operand
constexpr int kPQPastRecords = 0x7FFFFFF0;      // store offset that every descriptor drops

// Position in a workgroup's tile list: list index j, token tile mi and channel tile ni
// of the XCD's range.
struct PQTile {
  int64_t j;
  int mi, ni;
};

// Load descriptors of one tile's token rows (a) and channel rows (b).
struct PQSrc {
  __amdgpu_buffer_rsrc_t a, b;
};

template <bool kDump>
__global__ __launch_bounds__(512, 1) void w8a8_gemm_pq_kernel(const int8_t* __restrict__ qa, const float* __restrict__ sa,
                                                              const int8_t* __restrict__ w, const float* __restrict__ sw,
                                                              const _Float16* __restrict__ bias, int64_t m, int n, int k,
                                                              _Float16* __restrict__ out, int32_t* __restrict__ acc_out,
                                                              int64_t mt_count, int nt_count, int groups) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) char smem[kPQScale + 256 * 4 * 3 + 256 * 2];
  float* const s_sa = reinterpret_cast<float*>(smem + kPQScale);
  float* const s_sw = s_sa + 256;
  float* const s_b32 = s_sw + 256;
  _Float16* const s_b16 = reinterpret_cast<_Float16*>(s_b32 + 256);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = wave >> 2, q = wave & 3;

  // this workgroup's tiles: items local, local + wpx, ... of its XCD's list
  const int xcd = static_cast<int>(blockIdx.x & 7);
  const int64_t local = blockIdx.x >> 3, wpx = gridDim.x >> 3;
  const int parts = 8 / groups;
  const int cg = xcd % groups, part = xcd / groups;
  const int cpg = (nt_count + groups - 1) / groups;
  const int64_t mpp = (mt_count + parts - 1) / parts;
  const int nt_lo = cg * cpg, nt_hi = nt_count < nt_lo + cpg ? nt_count : nt_lo + cpg;
  const int ntg = nt_hi - nt_lo;
  const int64_t mt_lo = part * mpp, mt_hi = mt_count < mt_lo + mpp ? mt_count : mt_lo + mpp;
  if (ntg <= 0 || mt_hi <= mt_lo) return;
  const int64_t items = ntg * (mt_hi - mt_lo);
  if (local >= items) return;
  const int64_t count = (items - local + wpx - 1) / wpx;
  // Tile j of the list is item local + j wpx = (token tile mi, channel tile ni) of the
  // XCD's range; the walk steps (mi, ni) with scalar additions (no division in the loop).
  const int step_m = static_cast<int>(wpx / ntg), step_n = static_cast<int>(wpx % ntg);
  auto advance = [&](PQTile t) {
    t.j += 1;
    t.mi += step_m;
    t.ni += step_n;
    if (t.ni >= ntg) {
      t.ni -= ntg;
      t.mi += 1;
    }
    return t;
  };
  auto tile_m0 = [&](const PQTile& t) { return (mt_lo + t.mi) * 256; };
  auto tile_n0 = [&](const PQTile& t) { return (nt_lo + t.ni) * 256; };

  // load descriptors of a tile's token and channel rows (rows past the matrix read
  // zeros; a tile past the list gets empty descriptors)
  auto src_of = [&](const PQTile& t) {
    PQSrc r;
    if (t.j < count) {
      const int64_t m0 = tile_m0(t);
      const int n0 = tile_n0(t);
      const int rows_a = m - m0 < 256 ? static_cast<int>(m - m0) : 256;
      const int rows_b = n - n0 < 256 ? n - n0 : 256;
      r.a = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(qa + m0 * k), 0, rows_a * k, kRawBufferFlags);
      r.b = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(w + static_cast<int64_t>(n0) * k), 0, rows_b * k,
                                              kRawBufferFlags);
    } else {
      r.a = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(qa), 0, 0, kRawBufferFlags);
      r.b = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(w), 0, 0, kRawBufferFlags);
    }
    return r;
  };
  // scales and bias of a tile (the caller passes the last tile again in place of one
  // past the list): every wave issues exactly two loads; a missing bias reads zeros
  const __amdgpu_buffer_rsrc_t rs_a =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(sa), 0, static_cast<int>(m * 4), kRawBufferFlags);
  const __amdgpu_buffer_rsrc_t rs_w = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(sw), 0, n * 4, kRawBufferFlags);
  const __amdgpu_buffer_rsrc_t rs_b = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<_Float16*>(bias != nullptr ? bias : reinterpret_cast<const _Float16*>(g_zero_bias)), 0,
      bias != nullptr ? n * 2 : 0, kRawBufferFlags);
  // Per-lane values of the epilogue and the scale loads are rebuilt from the lane index
  // recomputed in place (volatile, so not hoisted), so that the compiler keeps nothing
  // of them live across the stage loop (where it would be spilled: a scratch reload is
  // a vector memory operation, and its wait would also wait for the ring loads).
  auto lane_now = []() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
  };
  auto load_scales = [&](const PQTile& t) {
    const int lane = lane_now();
    const int64_t m0 = tile_m0(t);
    const int n0 = tile_n0(t);
    if (wave < 4) {
      const int64_t r = m0 + wave * 64 + lane;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_a, lds_ptr(reinterpret_cast<char*>(s_sa) + wave * 256), 4,
                                               static_cast<int>(r < m ? r : m - 1) * 4, 0, 0, 0);
    } else {
      const int c = n0 + (wave - 4) * 64 + lane;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_w, lds_ptr(reinterpret_cast<char*>(s_sw) + (wave - 4) * 256), 4,
                                               (c < n ? c : n - 1) * 4, 0, 0, 0);
    }
    const int d = n0 / 2 + (wave & 1) * 64 + lane;  // bias dword: channels 2 d, 2 d + 1 (n is even)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_b, lds_ptr(reinterpret_cast<char*>(s_b16) + (wave & 1) * 256), 4,
                                             (d < n / 2 ? d : n / 2 - 1) * 4, 0, 0, 0);
  };

  const int c16 = ((lane & 3) ^ ((lane >> 4) & 3)) * 16;
  int vo[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) vo[j] = (128 * g + (2 * q + j) * 16 + (lane >> 2)) * k + c16;
  auto issue = [&](const PQSrc& r, int s, auto slc) {
    constexpr int SL = decltype(slc)::value;
#pragma unroll
    for (int j = 0; j < 2; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r.a, lds_ptr(smem + SL * kPPStage + (8 * g + 2 * q + j) * 1024), 16,
                                               vo[j], s * 64, 0, 0);
#pragma unroll
    for (int j = 0; j < 2; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r.b, lds_ptr(smem + SL * kPPStage + kPPHalf + (8 * g + 2 * q + j) * 1024),
                                               16, vo[j], s * 64, 0, 0);
  };

  u32x4 fw[2][2], fq[2][4];
  const char* bw[2][2];
  const char* bq[2][2];
#pragma unroll
  for (int G = 0; G < 2; ++G) {
    const int c = 2 * G + (lane >> 5);
    bw[G][0] = smem + kPPHalf + lds_off64(64 * q + (lane & 31), c);
    bq[G][0] = smem + lds_off64(128 * g + (lane & 31), c);
    bw[G][1] = bw[G][0] + 2 * kPPStage;
    bq[G][1] = bq[G][0] + 2 * kPPStage;
  }
  auto read_frags = [&](auto slc) {
    constexpr int SL = decltype(slc)::value;
#pragma unroll
    for (int G = 0; G < 2; ++G) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
        fw[G][nb] = *reinterpret_cast<const u32x4*>(bw[G][SL >> 1] + (SL & 1) * kPPStage + nb * 2048);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
        fq[G][mb] = *reinterpret_cast<const u32x4*>(bq[G][SL >> 1] + (SL & 1) * kPPStage + mb * 2048);
    }
  };
  i32x16 acc[2][4];
  auto compute = [&](auto first) {
    constexpr bool kFirst = decltype(first)::value;
    wait_lgkm0();
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int G = 0; G < 2; ++G)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          if (kFirst && G == 0)
            acc[nb][mb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, fw[G][nb]),
                                                              __builtin_bit_cast(i32x4, fq[G][mb]), i32x16{}, 0, 0, 0);
          else
            acc[nb][mb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, fw[G][nb]),
                                                              __builtin_bit_cast(i32x4, fq[G][mb]), acc[nb][mb], 0, 0, 0);
        }
    __builtin_amdgcn_s_setprio(0);
  };
  auto wait_n = [&](auto nn) {
    constexpr int N = decltype(nn)::value;
    wait_vmcnt<N>();
  };

  // Epilogue of the tile at (m0, n0): four rounds of 64 rows through ring slot 3.
  char* const C = smem + 3 * kPPStage;
  auto epilogue = [&](int64_t m0, int n0) {
    const int lane = lane_now(), tid = wave * 64 + lane;
    const int rows_a = m - m0 < 256 ? static_cast<int>(m - m0) : 256;
    const __amdgpu_buffer_rsrc_t ro =
        __builtin_amdgcn_make_buffer_rsrc(out + m0 * n, 0, rows_a * n * 2, kRawBufferFlags);
    const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(
        kDump ? acc_out + m0 * n : acc_out, 0, kDump ? rows_a * n * 4 : 0, kRawBufferFlags);
    const int srow = 32 * g + (lane & 31);  // staging row of this lane
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 128 * g + 32 * r + (lane & 31);
      const float sar = s_sa[row];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int col = 64 * q + nb * 32 + 8 * q4 + 4 * (lane >> 5);
          const f32x4 swv = *reinterpret_cast<const f32x4*>(s_sw + col);
          const f32x4 bv = *reinterpret_cast<const f32x4*>(s_b32 + col);
          _Float16 h[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            h[e] = static_cast<_Float16>((static_cast<float>(acc[nb][r][4 * q4 + e]) * sar) * swv[e] + bv[e]);
          // written through asm: the compiler cannot tell slot 3 from the slots that the
          // next tile's loads are filling and would wait for all of them first
          const uint32_t dst = lds_addr(C + srow * 512 + (((col >> 3) ^ (srow & 31)) << 4) + (col & 7) * 2);
          typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
          const u32x2 hv = __builtin_bit_cast(u32x2, h);
          asm volatile("ds_write_b64 %0, %1" ::"v"(dst), "v"(hv) : "memory");
          if constexpr (kDump) {
            const i32x4 v = {acc[nb][r][4 * q4], acc[nb][r][4 * q4 + 1], acc[nb][r][4 * q4 + 2], acc[nb][r][4 * q4 + 3]};
            const int off = n0 + col < n ? (row * n + n0 + col) * 4 : kPQPastRecords;
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rd, off, 0, 0);
          }
        }
      }
      if (r == 3 && g == 0) read_frags(std::integral_constant<int, 0>{});  // the next tile's stage 0
      wait_lgkm0();
      raw_barrier();
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int idx = i * 512 + tid;
        const int sr = idx >> 5, ch = idx & 31;
        const u32x4 v = *reinterpret_cast<const u32x4*>(C + sr * 512 + ((ch ^ (sr & 31)) << 4));
        const int trow = (sr < 32 ? 0 : 96) + 32 * r + sr;
        const int off = n0 + ch * 8 < n ? (trow * n + n0 + ch * 8) * 2 : kPQPastRecords;
        // nontemporal (cache policy NT): the fp16 output streams past L2 instead of
        // evicting the operand rows the next tiles read (shape A 357 -> 301 us)
        __builtin_amdgcn_raw_buffer_store_b128(v, ro, off, 0, kCachePolicyNT);
      }
      wait_lgkm0();
      raw_barrier();
    }
    if constexpr (kDump) wait_vmcnt<0>();
  };

  using SL0 = std::integral_constant<int, 0>;
  using SL1 = std::integral_constant<int, 1>;
  using SL2 = std::integral_constant<int, 2>;
  using SL3 = std::integral_constant<int, 3>;
  using Yes = std::true_type;
  using No = std::false_type;
  using W4 = std::integral_constant<int, 4>;
  using W8 = std::integral_constant<int, 8>;
  using WE0 = std::integral_constant<int, 4 + kPQEpiOps>;      // group 0, stages 0-1
  using WE1 = std::integral_constant<int, 8 + kPQEpiOps>;      // group 1, stages 0-1

  // Prologue: scales of tile 0, stages 0-2 of tile 0 from every wave, all complete.
  const int S = k >> 6;  // a multiple of 4, at least 8
  PQTile t0 = {0, static_cast<int>(local / ntg), static_cast<int>(local % ntg)};
  PQTile t1 = advance(t0);
  PQSrc cur = src_of(t0), nxt = src_of(t1);
  load_scales(t0);
  issue(cur, 0, SL0{});
  issue(cur, 1, SL1{});
  issue(cur, 2, SL2{});
  wait_vmcnt<0>();
  raw_barrier();
  if (g == 0) read_frags(SL0{});

  // Stage s of a tile: phase A(s), group 0 multiplies while group 1 issues its loads of
  // stage s + 3 and reads its fragments of s; phase B(s), group 1 multiplies while group
  // 0 issues its loads of s + 3 and reads its fragments of s + 1. Stage s + 3 belongs to
  // the next tile for s >= S - 3 (descriptor `nxt`, K offset s + 3 - S). Group 0 reads
  // the next tile's first fragments inside the epilogue, once its accumulators are
  // converted, so that both never hold registers at the same time.
  auto g0_stage = [&](const PQSrc& r, int s3, auto slc, auto wn, auto first, auto widen, auto readf) {
    constexpr int SL = decltype(slc)::value;
    __builtin_amdgcn_sched_barrier(0);
    compute(first);  // A(s)
    __builtin_amdgcn_sched_barrier(0);
    wait_n(wn);  // own loads of stage s + 1 landed
    raw_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue(r, s3, std::integral_constant<int, (SL + 3) & 3>{});  // B(s)
    if constexpr (decltype(readf)::value) read_frags(std::integral_constant<int, (SL + 1) & 3>{});
    if constexpr (decltype(widen)::value) {
      const int t = wave * 64 + lane_now();
      s_b32[t] = static_cast<float>(s_b16[t]);
    }
    __builtin_amdgcn_sched_barrier(0);
    raw_barrier();
  };
  auto g1_stage = [&](const PQSrc& r, int s3, auto slc, auto wn, auto first) {
    constexpr int SL = decltype(slc)::value;
    __builtin_amdgcn_sched_barrier(0);
    issue(r, s3, std::integral_constant<int, (SL + 3) & 3>{});  // A(s)
    read_frags(slc);
    __builtin_amdgcn_sched_barrier(0);
    wait_n(wn);
    raw_barrier();
    __builtin_amdgcn_sched_barrier(0);
    compute(first);  // B(s)
    __builtin_amdgcn_sched_barrier(0);
    raw_barrier();
  };

  // Each group runs its own copy of the tile loop (the branch on the group stays out of
  // the loop).
  auto tile_end = [&]() {
    epilogue(tile_m0(t0), tile_n0(t0));
    load_scales(t1.j < count ? t1 : t0);
    t0 = t1;
    t1 = advance(t1);
    cur = nxt;
    nxt = src_of(t1);
  };
  if (g == 0) {
    for (int64_t j = 0; j < count; ++j) {
      g0_stage(cur, 3, SL0{}, WE0{}, Yes{}, No{}, Yes{});
      g0_stage(cur, 4, SL1{}, WE0{}, No{}, No{}, Yes{});
      g0_stage(cur, 5, SL2{}, W4{}, No{}, No{}, Yes{});
      g0_stage(cur, 6, SL3{}, W4{}, No{}, Yes{}, Yes{});
      for (int s = 4; s < S - 4; s += 4) {
        g0_stage(cur, s + 3, SL0{}, W4{}, No{}, No{}, Yes{});
        g0_stage(cur, s + 4, SL1{}, W4{}, No{}, No{}, Yes{});
        g0_stage(cur, s + 5, SL2{}, W4{}, No{}, No{}, Yes{});
        g0_stage(cur, s + 6, SL3{}, W4{}, No{}, No{}, Yes{});
      }
      g0_stage(cur, S - 1, SL0{}, W4{}, No{}, No{}, Yes{});
      g0_stage(nxt, 0, SL1{}, W4{}, No{}, No{}, Yes{});
      g0_stage(nxt, 1, SL2{}, W4{}, No{}, No{}, Yes{});
      g0_stage(nxt, 2, SL3{}, W4{}, No{}, No{}, No{});
      tile_end();
    }
  } else {
    for (int64_t j = 0; j < count; ++j) {
      g1_stage(cur, 3, SL0{}, WE1{}, Yes{});
      g1_stage(cur, 4, SL1{}, WE1{}, No{});
      g1_stage(cur, 5, SL2{}, W8{}, No{});
      g1_stage(cur, 6, SL3{}, W8{}, No{});
      for (int s = 4; s < S - 4; s += 4) {
        g1_stage(cur, s + 3, SL0{}, W8{}, No{});
        g1_stage(cur, s + 4, SL1{}, W8{}, No{});
        g1_stage(cur, s + 5, SL2{}, W8{}, No{});
        g1_stage(cur, s + 6, SL3{}, W8{}, No{});
      }
      g1_stage(cur, S - 1, SL0{}, W8{}, No{});
      g1_stage(nxt, 0, SL1{}, W8{}, No{});
      g1_stage(nxt, 1, SL2{}, W8{}, No{});
      g1_stage(nxt, 2, SL3{}, W8{}, No{});
      tile_end();
    }
  }
  wait_vmcnt<0>();  // the loads past the list land before the workgroup's LDS is released
}

// Channel-tile groups of the ping-pong GEMM's tile order: the G (1, 2, 4 or 8, at most
// the channel-tile count) that minimises the operand bytes the XCDs fetch past their L2:
// token rows are fetched once per group, and channel rows once per XCD when the group's
// slice fits in half the 4 MB L2, else once per round of the token blocks an XCD holds
// in flight.
int pp_groups(int64_t mt, int nt, int k) {
  int best = 1;
  double best_cost = -1.0;
  for (int gr = 1; gr <= 8 && gr <= nt; gr *= 2) {
    const int parts = 8 / gr;
    const int64_t cpg = (nt + gr - 1) / gr;
    const int64_t mpp = (mt + parts - 1) / parts;
    const double b_xcd = static_cast<double>(cpg) * 256.0 * k;
    const int64_t in_flight = cpg >= 32 ? 1 : 32 / cpg;
    const int64_t rounds = (mpp + in_flight - 1) / in_flight;
    const double cost = static_cast<double>(mt) * 256.0 * k * gr + 8.0 * b_xcd * (b_xcd > (2 << 20) ? rounds : 1);
    if (best_cost < 0 || cost < best_cost) {
      best_cost = cost;
      best = gr;
    }
  }
  return best;
}

template <int NP>
void launch_quant(const _Float16* x, int64_t m, int k, const float* signs, int8_t* q, float* s, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(std::min<int64_t>(ceil_div(m, 4), int64_t(compute_units()) * 8)));
  const size_t lds = static_cast<size_t>(k) * sizeof(float);
  if (k % kQuantCols == 0) {
    if (signs) hipLaunchKernelGGL((quant_kernel<NP, true, true>), grid, dim3(256), lds, stream, x, m, k, signs, q, s);
    else hipLaunchKernelGGL((quant_kernel<NP, false, true>), grid, dim3(256), 0, stream, x, m, k, signs, q, s);
  } else {
    if (signs) hipLaunchKernelGGL((quant_kernel<NP, true, false>), grid, dim3(256), lds, stream, x, m, k, signs, q, s);
    else hipLaunchKernelGGL((quant_kernel<NP, false, false>), grid, dim3(256), 0, stream, x, m, k, signs, q, s);
  }
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
  if (signs) HI3D_REQUIRE((reinterpret_cast<uintptr_t>(signs) & 15) == 0, "multipliers must be 16-byte aligned");
  const int passes = (k + kQuantCols - 1) / kQuantCols;
  if (passes <= 1) launch_quant<1>(xh, m, k, signs, q, scale, stream);
  else if (passes <= 2) launch_quant<2>(xh, m, k, signs, q, scale, stream);
  else if (passes <= 4) launch_quant<4>(xh, m, k, signs, q, scale, stream);
  else if (passes <= 8) launch_quant<8>(xh, m, k, signs, q, scale, stream);
  else launch_quant<16>(xh, m, k, signs, q, scale, stream);
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
  const int64_t mtiles = ceil_div(m, kGemmBM);
  const int ntiles = static_cast<int>(ceil_div(n, kGemmBN));
  const int64_t blocks = mtiles * ntiles;
  HI3D_REQUIRE(blocks < (int64_t(1) << 31), "problem too large");
  const _Float16* b = static_cast<const _Float16*>(bias);
  _Float16* o = static_cast<_Float16*>(out);
  // per-lane source offsets within a 256-row tile are 32-bit
  // The persistent kernel removes the per-tile load latency and overlaps tiles; its stage
  // loop is slower than the one-tile kernel's, so it pays off for short K loops only
  // (measured: K = 1024 faster, K = 4096 slower).
  // The persistent ping-pong kernel takes K a multiple of 256 from 512 on with n % 8 == 0
  // and 32-bit byte offsets within a tile of the output (and of acc_out, 16-byte aligned,
  // whose int32 accumulators it also stores).
  const bool aligned4 = ((reinterpret_cast<uintptr_t>(sa) | reinterpret_cast<uintptr_t>(sw) |
                          reinterpret_cast<uintptr_t>(bias)) & 3) == 0 &&
                        (reinterpret_cast<uintptr_t>(acc_out) & 15) == 0;
  if (k % 256 == 0 && k >= 512 && n % 8 == 0 && static_cast<int64_t>(k) * 256 < (int64_t(1) << 31) &&
      m < (int64_t(1) << 29) &&
      static_cast<int64_t>(n) * (acc_out ? 1024 : 512) < (int64_t(1) << 31) - 4096 && aligned4) {
    const int gr = pp_groups(mtiles, ntiles, k);
    const int parts = 8 / gr;
    const int64_t per_xcd = static_cast<int64_t>((ntiles + gr - 1) / gr) * ((mtiles + parts - 1) / parts);
    const int cus = compute_units();
    HI3D_REQUIRE(cus > 0, "cannot query the compute unit count");
    const int64_t wpx = std::min<int64_t>(per_xcd, std::max(1, cus / 8));
    const dim3 grid(static_cast<unsigned>(wpx * 8));
    if (acc_out)
      hipLaunchKernelGGL(w8a8_gemm_pq_kernel<true>, grid, dim3(512), 0, stream, q, sa, w, sw, b, m, n, k, o, acc_out,
                         mtiles, ntiles, gr);
    else
      hipLaunchKernelGGL(w8a8_gemm_pq_kernel<false>, grid, dim3(512), 0, stream, q, sa, w, sw, b, m, n, k, o, acc_out,
                         mtiles, ntiles, gr);
    HI3D_LAUNCH_CHECK();
    return HI3D_OK;
  }
  // The ping-pong kernel takes K a multiple of 256 with n % 8 == 0 (with
  // acc_out it also stores the int32 accumulators, 16-byte aligned).
  if (k % 256 == 0 && n % 8 == 0 && static_cast<int64_t>(k) * 256 < (int64_t(1) << 31) &&
      (reinterpret_cast<uintptr_t>(sa) & 3) == 0 && (reinterpret_cast<uintptr_t>(sw) & 3) == 0 &&
      (reinterpret_cast<uintptr_t>(bias) & 3) == 0 && (reinterpret_cast<uintptr_t>(acc_out) & 15) == 0) {
    const int gr = pp_groups(mtiles, ntiles, k);
    const int parts = 8 / gr;
    const int64_t per_xcd = static_cast<int64_t>((ntiles + gr - 1) / gr) * ((mtiles + parts - 1) / parts);
    HI3D_REQUIRE(per_xcd * 8 < (int64_t(1) << 31), "problem too large");
    const dim3 grid(static_cast<unsigned>(per_xcd * 8));
    if (acc_out)
      hipLaunchKernelGGL(w8a8_gemm_pp_kernel<true>, grid, dim3(512), 0, stream, q, sa, w, sw, b, m, n, k, o, acc_out,
                         mtiles, ntiles, gr);
    else
      hipLaunchKernelGGL(w8a8_gemm_pp_kernel<false>, grid, dim3(512), 0, stream, q, sa, w, sw, b, m, n, k, o, acc_out,
                         mtiles, ntiles, gr);
    HI3D_LAUNCH_CHECK();
    return HI3D_OK;
  }
  // With acc_out the same kernel also stores the int32 accumulators (16-byte aligned).
  if (k % 64 == 0 && k >= 4 * 64 && k < 32 * 64 && m >= kGemmBM && n >= kGemmBN && n % 8 == 0 &&
      static_cast<int64_t>(kGemmBM) * k < (int64_t(1) << 32) && (reinterpret_cast<uintptr_t>(sa) & 3) == 0 &&
      (reinterpret_cast<uintptr_t>(sw) & 3) == 0 && (reinterpret_cast<uintptr_t>(bias) & 3) == 0 &&
      (reinterpret_cast<uintptr_t>(acc_out) & 15) == 0) {
    const int cus = compute_units();
    HI3D_REQUIRE(cus > 0, "cannot query the compute unit count");
    const int64_t workers = blocks < cus ? blocks : cus;
    if (acc_out)
      hipLaunchKernelGGL(w8a8_gemm_persistent_kernel<true>, dim3(static_cast<unsigned>(workers)), dim3(256), 0, stream,
                         q, sa, w, sw, b, m, n, k, o, acc_out, ntiles, blocks);
    else
      hipLaunchKernelGGL(w8a8_gemm_persistent_kernel<false>, dim3(static_cast<unsigned>(workers)), dim3(256), 0, stream,
                         q, sa, w, sw, b, m, n, k, o, acc_out, ntiles, blocks);
    HI3D_LAUNCH_CHECK();
    return HI3D_OK;
  }
  HI3D_REQUIRE(static_cast<int64_t>(kGemmBM) * k < (int64_t(1) << 32), "k too large");
  const dim3 grid(static_cast<unsigned>(blocks));
  if (k % 64 == 0) {
    if (acc_out)
      hipLaunchKernelGGL((w8a8_gemm_kernel<true, false>), grid, dim3(256), 0, stream, q, sa, w, sw, b, m, n, k, o, acc_out,
                         ntiles);
    else
      hipLaunchKernelGGL((w8a8_gemm_kernel<false, false>), grid, dim3(256), 0, stream, q, sa, w, sw, b, m, n, k, o,
                         acc_out, ntiles);
  } else {
    if (acc_out)
      hipLaunchKernelGGL((w8a8_gemm_kernel<true, true>), grid, dim3(256), 0, stream, q, sa, w, sw, b, m, n, k, o, acc_out,
                         ntiles);
    else
      hipLaunchKernelGGL((w8a8_gemm_kernel<false, true>), grid, dim3(256), 0, stream, q, sa, w, sw, b, m, n, k, o,
                         acc_out, ntiles);
  }
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

}  // extern "C"
