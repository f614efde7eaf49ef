// Gather-MFMA sparse convolution (submanifold 3^3, 2x2x2/s2 and its transpose) on gfx950.
//
//   out[o] = act(bias + sum_k in[table[o, k]] . W[:, k, :]^T) (+ residual[o])
//
// Reference semantics: subm_conv (src/hi3d_mac/torch_backend/sparse_conv.py:152-195),
// whose per-offset gather/matmul/index_add_ passes this kernel replaces by one
// output-stationary pass; sparse_conv (src/hi3d_mac/mlx_backend/sparse.py:191-214),
// which runs the dense 27-tap GEMM this kernel restricts to the offsets present.
//
// One workgroup (4 waves) owns a tile of kTileRows = 128 output rows (from the plan,
// see plan.hip) and BN output channels. For every (present offset k, 128-byte K-block)
// it gathers the 128 neighbour rows with 16-byte loads into LDS (absent rows become
// zeros), loads W[n0:n0+BN, k, K-block] and runs 32x32 MFMAs with fp32 accumulators in
// registers; stages are double-buffered (global loads of stage s+1 are in flight while
// stage s computes). The epilogue adds bias, applies SiLU, stages the tile through LDS
// and writes every output row exactly once with 16-byte stores (plus the residual).
#include <type_traits>
#include <utility>

#include "common.h"
#include "conv_tile.h"
#include "quant.h"
#include "rownorm.h"

namespace hi3d {
namespace {

struct ConvArgs {
  const char* in;
  int64_t n_in;
  int32_t cin;
  const char* weight;
  const void* bias;
  int32_t cout;
  int32_t kvol;
  const int32_t* rows;
  const int32_t* gidx;
  const uint32_t* tile_mask;
  int64_t ntiles;
  int64_t n_out;  // output rows (plan entries at or past it are not written)
  int32_t ny;  // column tiles
  const char* residual;
  int32_t act;
  char* out;
  // the row norm of conv_wide_kernel<.., kLN>: LayerNorm of each 128-channel output row,
  // then fp16(fp16(h * scale[b]) + shift[b]) and SiLU, b = the row's batch (coords[4 r])
  const int32_t* ln_coords;
  const void* ln_scale;  // fp16 [ln_batches, cout]
  const void* ln_shift;  // fp16 [ln_batches, cout]
  int32_t ln_batches;
  float ln_eps;
};

template <typename T>
__device__ __forceinline__ float to_f32(T v) {
  return static_cast<float>(v);
}

template <typename T, int BN>
__global__ __launch_bounds__(256) void conv_mfma_kernel(ConvArgs a) {
  constexpr int BM = kTileRows;
  constexpr int MB = 2;                 // 32-row blocks per wave (wave tile 64 rows)
  constexpr int WN = BN / 2;            // wave tile columns
  constexpr int NB = WN / 32;           // 32-column blocks per wave
  constexpr int A_BYTES = BM * 128;
  constexpr int B_BYTES = BN * 128;
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int PIPE = 2 * STAGE;
  constexpr int EPI = BM * BN * static_cast<int>(sizeof(T));
  constexpr int SMEM = PIPE > EPI ? PIPE : EPI;
  constexpr int BL = BN / 32;           // B chunks loaded per thread per stage
  __shared__ __attribute__((aligned(16))) char smem[SMEM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t item = xcd_remap(blockIdx.x, static_cast<int64_t>(gridDim.x));
  const int64_t tile = item / a.ny;
  const int n0 = static_cast<int>(item % a.ny) * BN;

  const int kvol = a.kvol;
  uint32_t mask = a.tile_mask[tile];
  if (kvol < 32) mask &= (1u << kvol) - 1u;
  const int row_bytes = a.cin * static_cast<int>(sizeof(T));
  const int row_chunks = row_bytes >> 4;
  const int nkb = (row_chunks + 7) >> 3;
  const int ntaps = kvol <= 32 ? __popc(mask) : kvol;
  const int S = ntaps * nkb;

  const int ld_row = tid >> 3, ld_chunk = tid & 7;
  const int32_t* gbase = a.gidx + tile * static_cast<int64_t>(kvol) * BM;
  const uint64_t n_in = static_cast<uint64_t>(a.n_in);

  u32x4 ra[4], rb[BL];
  const u32x4 zero = {0u, 0u, 0u, 0u};

  // load iterator over (tap, K-block)
  int lk = kvol <= 32 ? (mask ? __builtin_ctz(mask) : 0) : 0;
  int lkb = 0;
  uint32_t lrest = kvol <= 32 ? (mask & (mask - 1u)) : 0u;

  auto load = [&]() {
    const int c = lkb * 8 + ld_chunk;
    const bool cok = c < row_chunks;
    const int32_t* g = gbase + lk * BM;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int32_t src = g[ld_row + 32 * i];
      ra[i] = (cok && static_cast<uint64_t>(static_cast<uint32_t>(src)) < n_in)
                  ? *reinterpret_cast<const u32x4*>(a.in + static_cast<int64_t>(src) * row_bytes + c * 16)
                  : zero;
    }
#pragma unroll
    for (int j = 0; j < BL; ++j) {
      const int n = n0 + ld_row + 32 * j;
      rb[j] = (cok && n < a.cout)
                  ? *reinterpret_cast<const u32x4*>(a.weight + (static_cast<int64_t>(n) * kvol + lk) * row_bytes + c * 16)
                  : zero;
    }
    if (++lkb == nkb) {
      lkb = 0;
      if (kvol <= 32) {
        lk = lrest ? __builtin_ctz(lrest) : lk;
        lrest &= lrest - 1u;
      } else {
        ++lk;
      }
    }
  };
  auto store = [&](int buf) {
    char* A = smem + buf * STAGE;
    char* B = A + A_BYTES;
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(A + lds_offset(ld_row + 32 * i, ld_chunk)) = ra[i];
#pragma unroll
    for (int j = 0; j < BL; ++j) *reinterpret_cast<u32x4*>(B + lds_offset(ld_row + 32 * j, ld_chunk)) = rb[j];
  };

  f32x16 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mb][nb][v] = 0.0f;

  auto compute = [&](int buf) {
    const char* A = smem + buf * STAGE;
    const char* B = A + A_BYTES;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c = 2 * g + (lane >> 5);
      u32x4 af[MB], bf[NB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        af[mb] = *reinterpret_cast<const u32x4*>(A + lds_offset(wm * 64 + mb * 32 + (lane & 31), c));
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        bf[nb] = *reinterpret_cast<const u32x4*>(B + lds_offset(wn * WN + nb * 32 + (lane & 31), c));
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) Mfma<T>::run(af[mb], bf[nb], acc[mb][nb]);
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

  // epilogue: bias + activation in fp32, round to T, stage the tile in LDS
  T* C = reinterpret_cast<T*>(smem);
  const T* bias = static_cast<const T*>(a.bias);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int j = wn * WN + nb * 32 + (lane & 31);
    const int n = n0 + j;
    const float b = (bias != nullptr && n < a.cout) ? to_f32(bias[n]) : 0.0f;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int i = wm * 64 + mb * 32 + acc_row(lane, v);
        float x = acc[mb][nb][v] + b;
        if (a.act == HI3D_ACT_SILU) x = silu_f32(x);
        C[i * BN + j] = static_cast<T>(x);
      }
    }
  }
  __syncthreads();
  constexpr int EPC = 16 / static_cast<int>(sizeof(T));  // elements per 16-byte chunk
  constexpr int CPR = BN / EPC;                            // chunks per tile row
  const int64_t out_row_bytes = static_cast<int64_t>(a.cout) * sizeof(T);
  for (int q = tid; q < BM * CPR; q += 256) {
    const int i = q / CPR, cc = q - (q / CPR) * CPR;
    const int32_t orow = a.rows[tile * BM + i];
    const int ncol = n0 + cc * EPC;
    if (orow < 0 || orow >= a.n_out || ncol >= a.cout) continue;
    u32x4 v = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(C) + (i * BN + cc * EPC) * sizeof(T));
    const int64_t off = static_cast<int64_t>(orow) * out_row_bytes + static_cast<int64_t>(ncol) * sizeof(T);
    if (a.residual != nullptr) {
      v = add_chunk<T>(v, *reinterpret_cast<const u32x4*>(a.residual + off));
    }
    *reinterpret_cast<u32x4*>(a.out + off) = v;
  }
}

// ------------------------------------------------------------------------------------
// Pipelined variant for kernel volumes up to 27 (3^3 submanifold, 2^3 strided pair).
//
// 8 waves (two per SIMD) share a BM x BN tile (64 x 64 per wave; 32 x 64 for BN = 64).
// Stages are (present offset, 128-byte K-block) pairs, so every gathered row moves as
// whole 128-byte lines. Global loads run three stages ahead into a ring of three
// register sets (16-byte loads; absent rows and K padding read a zero buffer); after
// computing stage s from LDS, a thread waits for its stage s+1 loads only (stages s+2
// and s+3 stay in flight), writes them to the other LDS buffer and joins a barrier. Fragment reads wait
// on the LDS counter only, never on in-flight global loads, and run two K-groups ahead
// of the MFMAs. The MFMAs take the weights as their first operand, so each lane's
// accumulators hold four consecutive output channels of one output row, staged for the
// epilogue with 8-byte LDS writes. The tile's gather indices (all offsets, [K][BM]) and
// output rows are copied to LDS once per tile; gather indices are read into registers
// once per offset. A stage's global loads are issued between its MFMA groups. A BM-row tile
// covers BM / 128 consecutive plan tiles (union of their masks).

__device__ __attribute__((aligned(16))) const uint32_t g_zero16[4] = {0u, 0u, 0u, 0u};

constexpr int kMaxPipelinedKvol = 27;
constexpr int kPipeThreads = 512;
constexpr int kRing = 3;  // register sets of in-flight global loads

template <typename T, int BM, int BN, int WGM>
__global__ __launch_bounds__(kPipeThreads) void conv_pipe_kernel(ConvArgs a) {
  constexpr int WGN = kPipeThreads / 64 / WGM;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int MB = WM / 32, NB = WN / 32;  // 32 x 32 blocks per wave
  static_assert(MB >= 1 && NB >= 1 && WGM * WGN == kPipeThreads / 64, "wave grid");
  constexpr int A_INS = BM / 64, B_INS = BN / 64;  // 16-byte loads per thread per stage
  constexpr int L = A_INS + B_INS;
  constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128;
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int PIPE = 2 * STAGE;
  constexpr int EPI = BM * BN * static_cast<int>(sizeof(T));
  constexpr int REGION = PIPE > EPI ? PIPE : EPI;
  constexpr int SUB = BM / kTileRows;
  __shared__ __attribute__((aligned(16))) char smem[REGION + BM * (kMaxPipelinedKvol + 1) * 4];
  int32_t* const gidx = reinterpret_cast<int32_t*>(smem + REGION);
  int32_t* const orows = gidx + BM * kMaxPipelinedKvol;  // output row of each tile slot

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int64_t item = xcd_remap(blockIdx.x, static_cast<int64_t>(gridDim.x));
  const int64_t tile = item / a.ny;
  const int n0 = static_cast<int>(item % a.ny) * BN;
  const int kvol = a.kvol;
  const int32_t absent = static_cast<int32_t>(a.n_in);

  uint32_t mask = 0;
#pragma unroll
  for (int h = 0; h < SUB; ++h) {
    const int64_t pt = tile * SUB + h;
    if (pt < a.ntiles) mask |= a.tile_mask[pt];
  }
  mask &= (1u << kvol) - 1u;

  // gather indices of the tile, all offsets: LDS [k][BM]; output rows: LDS [BM]
  for (int i = tid; i < BM; i += kPipeThreads) {
    const int64_t pt = tile * SUB + i / kTileRows;
    orows[i] = pt < a.ntiles ? a.rows[pt * kTileRows + (i % kTileRows)] : -1;
  }
  {
    const int per_k = BM / 4;
    for (int q = tid; q < kvol * per_k; q += kPipeThreads) {
      const int k = q / per_k;
      const int r = (q - k * per_k) * 4;
      const int64_t pt = tile * SUB + r / kTileRows;
      i32x4 v = {absent, absent, absent, absent};
      if (pt < a.ntiles) v = *reinterpret_cast<const i32x4*>(a.gidx + (pt * kvol + k) * kTileRows + (r % kTileRows));
      *reinterpret_cast<i32x4*>(gidx + k * BM + r) = v;
    }
  }
  __syncthreads();

  const int row_bytes = a.cin * static_cast<int>(sizeof(T));
  const int row_chunks = row_bytes >> 4;
  const int nkb = (row_chunks + 7) >> 3;
  const int S = __popc(mask) * nkb;
  const uint64_t n_in = static_cast<uint64_t>(a.n_in);
  const int lrow = tid >> 3, lchunk = tid & 7;  // this thread loads rows lrow + 64 j, chunk lchunk

  int ik = mask ? __builtin_ctz(mask) : 0, ikb = 0;
  uint32_t irest = mask & (mask - 1u);
  int32_t asrc[A_INS];
  u32x4 ra[kRing][A_INS], rb[kRing][B_INS];

  auto load_a = [&](const int r) {
    if (ikb == 0) {
      const int32_t* g = gidx + ik * BM;
#pragma unroll
      for (int j = 0; j < A_INS; ++j) asrc[j] = g[lrow + 64 * j];
    }
    const int cidx = ikb * 8 + lchunk;
    const bool cok = cidx < row_chunks;
#pragma unroll
    for (int j = 0; j < A_INS; ++j) {
      const int32_t src = asrc[j];
      const bool ok = cok && static_cast<uint64_t>(static_cast<uint32_t>(src)) < n_in;
      const char* real = a.in + static_cast<int64_t>(ok ? src : 0) * row_bytes + cidx * 16;
      ra[r][j] = *reinterpret_cast<const u32x4*>(ok ? static_cast<const void*>(real) : static_cast<const void*>(g_zero16));
    }
  };
  auto load_b = [&](const int r) {
    const int cidx = ikb * 8 + lchunk;
    const bool cok = cidx < row_chunks;
#pragma unroll
    for (int j = 0; j < B_INS; ++j) {
      const int n = n0 + lrow + 64 * j;
      const bool ok = cok && n < a.cout;
      const char* real = a.weight + (static_cast<int64_t>(ok ? n : 0) * kvol + ik) * row_bytes + cidx * 16;
      rb[r][j] = *reinterpret_cast<const u32x4*>(ok ? static_cast<const void*>(real) : static_cast<const void*>(g_zero16));
    }
    if (++ikb == nkb) {
      ikb = 0;
      ik = irest ? __builtin_ctz(irest) : ik;
      irest &= irest - 1u;
    }
  };
  auto store = [&](const int r, const int buf) {
    char* A = smem + buf * STAGE;
    char* B = A + A_BYTES;
#pragma unroll
    for (int j = 0; j < A_INS; ++j) *reinterpret_cast<u32x4*>(A + lds_offset(lrow + 64 * j, lchunk)) = ra[r][j];
#pragma unroll
    for (int j = 0; j < B_INS; ++j) *reinterpret_cast<u32x4*>(B + lds_offset(lrow + 64 * j, lchunk)) = rb[r][j];
  };

  // acc[nb][mb]: channels block nb (MFMA rows) x output-row block mb (MFMA columns)
  f32x16 acc[NB][MB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[nb][mb][v] = 0.0f;

  auto load = [&](const int r) {
    load_a(r);
    load_b(r);
  };

  // compute stage `buf` from LDS; with `issue` set, the global loads of the next stage
  // for register set `next` (a compile-time constant) are issued between the MFMA groups
  // so a stalled load issue overlaps MFMAs already in flight
  auto compute = [&](const int buf, auto nc, const bool issue) {
    constexpr int next = decltype(nc)::value;
    const char* A = smem + buf * STAGE;
    const char* B = A + A_BYTES;
    u32x4 af[4][MB], bf[4][NB];
    auto frags = [&](int g) {
      const int c = 2 * g + (lane >> 5);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        af[g][mb] = *reinterpret_cast<const u32x4*>(A + lds_offset(wm * WM + mb * 32 + (lane & 31), c));
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        bf[g][nb] = *reinterpret_cast<const u32x4*>(B + lds_offset(wn * WN + nb * 32 + (lane & 31), c));
    };
    auto mma = [&](int g) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) Mfma<T>::run(bf[g][nb], af[g][mb], acc[nb][mb]);
    };
    frags(0);
    frags(1);
    __builtin_amdgcn_sched_barrier(0);
    mma(0);
    __builtin_amdgcn_sched_barrier(0);
    if (issue) load_a(next);
    __builtin_amdgcn_sched_barrier(0);
    frags(2);
    __builtin_amdgcn_sched_barrier(0);
    mma(1);
    __builtin_amdgcn_sched_barrier(0);
    if (issue) load_b(next);
    __builtin_amdgcn_sched_barrier(0);
    frags(3);
    __builtin_amdgcn_sched_barrier(0);
    mma(2);
    __builtin_amdgcn_sched_barrier(0);
    mma(3);
  };

  // one pipeline step; R = s % kRing and the LDS buffer s & 1 are compile-time
  // constants (the loop is unrolled by 2 * kRing) so every register set stays in
  // registers. Stage s+kRing is loaded into the set that held stage s; stages
  // s+1 .. s+kRing are in flight while stage s computes.
  auto step = [&](int s, auto rc, auto bc) {
    constexpr int R = decltype(rc)::value, BUF = decltype(bc)::value;
    constexpr int RN = (R + 1) % kRing;
    compute(BUF, rc, s + kRing < S);
    if (s + 1 < S) {
      const int newer = (S - 2 - s) < (kRing - 1) ? (S - 2 - s) : (kRing - 1);  // stages issued after s+1
      if (newer >= 2) wait_vmcnt<2 * L>();
      else if (newer == 1) wait_vmcnt<L>();
      else wait_vmcnt<0>();
      __builtin_amdgcn_sched_barrier(0);
      store(RN, 1 - BUF);
      wait_lgkm0();
    }
    __builtin_amdgcn_s_barrier();
  };
  if (S > 0) {
#pragma unroll
    for (int r = 0; r < kRing; ++r)
      if (r < S) load(r);
    const int newer = (S - 1) < (kRing - 1) ? (S - 1) : (kRing - 1);
    if (newer >= 2) wait_vmcnt<2 * L>();
    else if (newer == 1) wait_vmcnt<L>();
    else wait_vmcnt<0>();
    store(0, 0);
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
  }
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  static_assert(kRing == 3, "the unrolled loop below is written for three register sets");
  for (int s = 0; s < S; s += 6) {
    step(s, I0{}, I0{});
    if (s + 1 < S) step(s + 1, I1{}, I1{});
    if (s + 2 < S) step(s + 2, I2{}, I0{});
    if (s + 3 < S) step(s + 3, I0{}, I1{});
    if (s + 4 < S) step(s + 4, I1{}, I0{});
    if (s + 5 < S) step(s + 5, I2{}, I1{});
  }
  __syncthreads();

  // epilogue: bias + activation in fp32, round to T; lane (l % 32) of block (nb, mb)
  // holds output row wm*WM + mb*32 + l%32 and channels wn*WN + nb*32 + 8*(v/4) +
  // 4*(l/32) + v%4: four consecutive channels per 8-byte LDS write
  T* C = reinterpret_cast<T*>(smem);
  const T* bias = static_cast<const T*>(a.bias);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int j0 = wn * WN + nb * 32 + 8 * q + 4 * (lane >> 5);
      float b[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int n = n0 + j0 + e;
        b[e] = (bias != nullptr && n < a.cout) ? to_f32(bias[n]) : 0.0f;
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int i = wm * WM + mb * 32 + (lane & 31);
        T h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float x = acc[nb][mb][4 * q + e] + b[e];
          if (a.act == HI3D_ACT_SILU) x = silu_f32(x);
          h[e] = static_cast<T>(x);
        }
        if constexpr (sizeof(T) == 2) {
          uint2 packed;
          __builtin_memcpy(&packed, h, 8);
          *reinterpret_cast<uint2*>(C + i * BN + j0) = packed;
        } else {
          u32x4 packed;
          __builtin_memcpy(&packed, h, 16);
          *reinterpret_cast<u32x4*>(C + i * BN + j0) = packed;
        }
      }
    }
  }
  __syncthreads();
  constexpr int EPC = 16 / static_cast<int>(sizeof(T));
  constexpr int CPR = BN / EPC;
  const int64_t out_row_bytes = static_cast<int64_t>(a.cout) * sizeof(T);
  for (int q = tid; q < BM * CPR; q += kPipeThreads) {
    const int i = q / CPR, cc = q - (q / CPR) * CPR;
    const int32_t orow = orows[i];
    const int ncol = n0 + cc * EPC;
    if (orow < 0 || orow >= a.n_out || ncol >= a.cout) continue;
    u32x4 v = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(C) + (i * BN + cc * EPC) * sizeof(T));
    const int64_t off = static_cast<int64_t>(orow) * out_row_bytes + static_cast<int64_t>(ncol) * sizeof(T);
    if (a.residual != nullptr) {
      v = add_chunk<T>(v, *reinterpret_cast<const u32x4*>(a.residual + off));
    }
    *reinterpret_cast<u32x4*>(a.out + off) = v;
  }
}

template <typename T, typename Acc>
__global__ void conv_simple_kernel(const T* __restrict__ in, int64_t n_in, int cin, const T* __restrict__ w,
                                   const T* __restrict__ bias, int cout, int kvol, const int32_t* __restrict__ table,
                                   int64_t n_out, const T* __restrict__ residual, int act, T* __restrict__ out) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= n_out * cout) return;
  const int64_t o = idx / cout;
  const int n = static_cast<int>(idx - o * cout);
  Acc acc = 0;
  for (int k = 0; k < kvol; ++k) {
    const int32_t src = table[o * kvol + k];
    if (static_cast<uint64_t>(static_cast<uint32_t>(src)) >= static_cast<uint64_t>(n_in)) continue;
    const T* x = in + static_cast<int64_t>(src) * cin;
    const T* wk = w + (static_cast<int64_t>(n) * kvol + k) * cin;
    for (int c = 0; c < cin; ++c) acc += static_cast<Acc>(x[c]) * static_cast<Acc>(wk[c]);
  }
  if (bias != nullptr) acc += static_cast<Acc>(bias[n]);
  if (act == HI3D_ACT_SILU) acc = acc / (static_cast<Acc>(1) + exp(-acc));
  T r = static_cast<T>(acc);
  if (residual != nullptr) r = static_cast<T>(static_cast<Acc>(r) + static_cast<Acc>(residual[idx]));
  out[idx] = r;
}

int elem_size(int dtype) {
  switch (dtype) {
    case HI3D_F32: return 4;
    case HI3D_F16: return 2;
    case HI3D_BF16: return 2;
    case HI3D_F64: return 8;
    default: return 0;
  }
}

// ------------------------------------------------------------- ring kernel --
// Gather convolution for fp16 / bf16 with Cout a multiple of 128, 256..512-byte input
// rows (4..8 steps of 64 bytes per offset) and at most 27 offsets: the submanifold
// 3x3x3 layers of 128 and 256 channels.
//  * Tile: BM output rows (the union of BM / 128 plan tiles' offset masks) x BN output
//    channels. NW waves (two per SIMD at NW = 8) form a 4 x NW / 4 grid; each owns
//    BM / 4 rows x 4 BN / NW channels as blocks of 32x32x16 MFMAs with the weights as the
//    first operand. BN = 128 takes BM = 384; BN = 256 (Cout a multiple of 256) takes
//    BM = 256, half the gathered bytes per flop of the 128-channel tile.
//  * Stages: (present offset, 64-byte K step). A stage is BM gathered rows + BN weight
//    rows of 64 bytes (32 KB) in a 4-deep LDS ring, filled by direct-to-LDS 16-byte loads
//    issued three stages ahead: per wave L = (BM + BN) / (16 NW) loads per stage, half in
//    the second half of stage s (cursor X) and half in the first half of stage s + 1
//    (cursor Y), each after one MFMA. Rows use the 64-byte swizzled layout of the int8
//    GEMM; absent neighbours load from a zero row.
//  * Gather indices: the tile's BM indices of an offset reach a two-slot LDS ring by
//    direct-to-LDS loads (some repeated so that every wave issues the same number),
//    issued when cursor X enters the previous offset; each cursor turns its rows'
//    indices into source addresses once per offset. The tile's output rows arrive the
//    same way at the start.
//  * One barrier per stage, between its two K-groups. Every wave issues the same loads,
//    so the vmcnt waits are exact: at the barrier of stage s the operations issued after
//    stage s + 1's last load are stage s + 2's L loads plus the index loads when stage
//    s + 2 begins an offset that has a successor.
//  * Epilogue: bias + activation in fp32, round to T; each wave stages its own block in
//    LDS and writes it as 16-byte row chunks to the tile's output rows, adding the
//    residual.
// Tile shapes: BN = 128 takes BM = 384 rows, BN = 256 takes 256 rows (32 KB stages);
// NW waves form a 4 x NW / 4 grid over rows x channels.
template <int BN, int NW, int BMv = (BN == 128 ? 384 : 256)>
struct RingShape {
  static constexpr int BM = BMv;
  static constexpr int SUB = BM / kTileRows;  // plan tiles per tile
  static constexpr int WM = 4, WN = NW / 4;   // wave grid
  static constexpr int MB = BM / WM / 32;     // row blocks per wave
  static constexpr int NB = BN / WN / 32;     // channel blocks per wave
  static constexpr int LA = BM / (16 * NW);   // gathered-row loads per wave and stage
  static constexpr int LB = BN / (16 * NW);   // weight-row loads per wave and stage
  static constexpr int L = LA + LB;
  static constexpr int STAGE_A = BM * 64;
  static constexpr int STAGE = STAGE_A + BN * 64;
  static constexpr int IDX = BM * 4;
  static constexpr int NIDX = BM / 64;        // 64-entry index loads of one offset
  static constexpr int IDXL = (NIDX + NW - 1) / NW;  // index loads per wave
};
constexpr int kRingDepth = 4;
constexpr int kRingMaxRowBytes = 2048;  // the zero row absent neighbours read is this long

__device__ __attribute__((aligned(16))) const uint32_t g_zero_row[kRingMaxRowBytes / 4] = {};

__device__ __forceinline__ void lds_dma4(const void* src, char* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(lds_wave_base), 4, 0, 0);
}

// source address of gathered row g (rows outside [0, n_in) read the zero row); the
// address is made opaque before the select so that it stays a v_cndmask, not a branch
__device__ __forceinline__ const char* gather_src(const char* in, int32_t g, uint64_t n_in, int rb, int coff,
                                                  const char* zrow) {
  const bool ok = static_cast<uint64_t>(static_cast<uint32_t>(g)) < n_in;
  uint64_t pin = reinterpret_cast<uint64_t>(in) + static_cast<uint64_t>(static_cast<int64_t>(g) * rb + coff);
  asm volatile("" : "+v"(pin));
  return ok ? reinterpret_cast<const char*>(pin) : zrow;
}

__device__ __forceinline__ int ring_off(int row, int chunk) {
  return row * 64 + ((chunk ^ ((row >> 2) & 3)) << 4);
}

template <typename T, int BN, int NW, int BMv>
__global__ __launch_bounds__(NW * 64, 1) void conv_ring_kernel(ConvArgs a) {
  using Sh = RingShape<BN, NW, BMv>;
  constexpr int NS = kRingDepth, BM = Sh::BM, MB = Sh::MB, NB = Sh::NB, LA = Sh::LA, L = Sh::L;
  constexpr int SUB = Sh::SUB, STAGE_A = Sh::STAGE_A, STAGE = Sh::STAGE, IDX = Sh::IDX;
  constexpr int IDXL = Sh::IDXL, LX = L / 2;  // cursor X issues loads 0..LX-1, Y the rest
  constexpr int RING = NS * STAGE;
  static_assert(STAGE % 1024 == 0 && LA * 16 * NW == BM && Sh::LB * 16 * NW == BN, "stage shape");
  // the epilogue stages the whole output tile over the ring; past it lie the tile's
  // output rows, which the stores read
  static_assert(BM * BN * static_cast<int>(sizeof(T)) <= RING, "output tile must fit the ring");
  constexpr int kBiasDwords = BN * static_cast<int>(sizeof(T)) / 4;
  constexpr int kBiasBytes = (kBiasDwords + 63) / 64 * 256;
  // one LDS array (a second one makes the compiler wait for every direct-to-LDS load
  // before each LDS read); the tile's bias sits at its end
  __shared__ __attribute__((aligned(16))) char smem[RING + 3 * IDX + 256 + kBiasBytes];
  char* const s_bias = smem + (RING + 3 * IDX + 256);
  char* const idx_ring = smem + RING;
  char* const rows_lds = idx_ring + 2 * IDX;  // the tile's output rows
  char* const idx_dummy = rows_lds + IDX;     // target of the index DMAs of stages entering no offset

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % Sh::WM, wn = wave / Sh::WM;
  const int64_t item = xcd_remap(blockIdx.x, static_cast<int64_t>(gridDim.x));
  const int64_t tile = item / a.ny;
  const int n0 = static_cast<int>(item - tile * a.ny) * BN;
  // the tile's bias reaches LDS by 4-byte DMAs before any stage is requested: the
  // oldest loads, so the stage loop's constant waits still hold, and no register waits
  // on them (the epilogue reads it after its wait for every load)
  if (a.bias != nullptr && wave < (kBiasDwords + 63) / 64) {
    const int d = wave * 64 + lane;
    lds_dma4(static_cast<const char*>(a.bias) + static_cast<int64_t>(n0) * sizeof(T) + 4 * (d < kBiasDwords ? d : kBiasDwords - 1),
             s_bias + wave * 256);
  }
  const int kvol = a.kvol;
  uint32_t mask = 0;
#pragma unroll
  for (int h = 0; h < SUB; ++h) {
    const int64_t pt = tile * SUB + h;
    if (pt < a.ntiles) mask |= a.tile_mask[pt];
  }
  mask &= (1u << kvol) - 1u;
  const int rb = a.cin * static_cast<int>(sizeof(T));
  const int KB = rb >> 6;
  const int taps = __popc(mask);
  const int S = taps * KB;
  const uint64_t n_in = static_cast<uint64_t>(a.n_in);

  // load u of this wave covers stage rows (wave + NW u) * 16 + lane / 4 (gathered rows for
  // u < LA, weight rows for u - LA after), at physical chunk lane % 4, i.e. logical chunk
  // `coff` / 16 (the swizzle repeats every 16 rows)
  const int r0 = wave * 16 + (lane >> 2);
  const int coff = ((lane & 3) ^ ((r0 >> 2) & 3)) * 16;
  const char* wrow[Sh::LB];
#pragma unroll
  for (int j = 0; j < Sh::LB; ++j)
    wrow[j] = a.weight + static_cast<int64_t>(n0 + r0 + 16 * NW * j) * kvol * rb + coff;
  const char* const zrow = reinterpret_cast<const char*>(g_zero_row) + coff;

  // 64-entry index loads: load i of NIDX covers rows 64 i .. +63 (plan tile i / 2, clamped
  // to the plan); wave w issues loads w, w + NW, ... (repeating its first beyond NIDX)
  auto idx_load = [&](const int32_t* base, int64_t stride, int u) {
    int i = wave + NW * u;
    if (i >= Sh::NIDX) i = wave < Sh::NIDX ? wave : Sh::NIDX - 1;
    int64_t pt = tile * SUB + (i >> 1);
    if (pt >= a.ntiles) pt = a.ntiles - 1;
    return std::pair<const int32_t*, int>(base + pt * stride + (i & 1) * 64 + lane, i * 256);
  };
  auto issue_idx = [&](int k, int slot) {
#pragma unroll
    for (int u = 0; u < IDXL; ++u) {
      auto [src, off] = idx_load(a.gidx + k * kTileRows, static_cast<int64_t>(kvol) * kTileRows, u);
      lds_dma4(src, idx_ring + slot * IDX + off);
    }
  };
  // the tile's output rows reach LDS at the start (complete by the first wait)
#pragma unroll
  for (int u = 0; u < IDXL; ++u) {
    auto [src, off] = idx_load(a.rows, kTileRows, u);
    lds_dma4(src, rows_lds + off);
  }

  // load cursors over the stage stream (present offsets in increasing order, K steps
  // inside); X issues loads 0..LX-1 of a stage, Y loads LX..L-1
  struct Cursor {
    uint32_t rest;  // offsets after the current one
    int k, kb, ord, slot;
    const char* src[LA];  // gathered-row sources of this cursor's loads at step 0
  };
  auto enter_offset = [&](Cursor& c, auto yc) {
    constexpr bool Y = decltype(yc)::value;
    constexpr int U0 = Y ? LX : 0, U1 = Y ? (LA < L ? LA : L) : (LA < LX ? LA : LX);
    const int32_t* gi = reinterpret_cast<const int32_t*>(idx_ring + (c.ord & 1) * IDX);
    int32_t g[LA];
#pragma unroll
    for (int u = U0; u < U1; ++u) g[u] = gi[r0 + 16 * NW * u];
#pragma unroll
    for (int u = U0; u < U1; ++u) c.src[u] = gather_src(a.in, g[u], n_in, rb, coff, zrow);
  };
  using XC = std::false_type;
  using YC = std::true_type;
  auto start = [&](Cursor& c) {
    c.k = mask ? __builtin_ctz(mask) : 0;
    c.rest = mask & (mask - 1u);
    c.kb = 0;
    c.ord = 0;
    c.slot = 0;
  };
  // advance to the next stage; returns true when it enters a new offset
  auto advance = [&](Cursor& c) {
    c.slot = (c.slot + 1) & (NS - 1);
    if (++c.kb == KB) {
      c.kb = 0;
      c.k = c.rest ? __builtin_ctz(c.rest) : c.k;
      c.rest &= c.rest - 1u;
      ++c.ord;
      return true;
    }
    return false;
  };
  auto issue = [&](Cursor& c, int u) {  // load u of the cursor's current stage
    char* st = smem + c.slot * STAGE;
    if (u < LA)
      lds_dma16(c.src[u] + c.kb * 64, st + (wave + NW * u) * 1024);
    else
      lds_dma16(wrow[u - LA] + c.k * rb + c.kb * 64, st + STAGE_A + (wave + NW * (u - LA)) * 1024);
  };

  f32x16 acc[NB][MB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[nb][mb][v] = 0.0f;
  constexpr int NF = NB + MB;  // fragment reads per K-group
  constexpr int NM = NB * MB;  // MFMAs per K-group
  static_assert(NM >= L - LX && NM >= LX, "slots");
  u32x4 fa[2][MB], fb[2][NB];
  auto frag_one = [&](int slot, auto gc, int i) {  // i: weight blocks, then row blocks
    constexpr int Gk = decltype(gc)::value;
    const char* st = smem + slot * STAGE;
    const int c = 2 * Gk + (lane >> 5);
    if (i < NB)
      fb[Gk][i] = *reinterpret_cast<const u32x4*>(st + STAGE_A + ring_off(wn * NB * 32 + i * 32 + (lane & 31), c));
    else
      fa[Gk][i - NB] =
          *reinterpret_cast<const u32x4*>(st + ring_off(wm * (MB * 32) + (i - NB) * 32 + (lane & 31), c));
  };
  auto mma_one = [&](auto gc, int i) {  // i = nb * MB + mb
    constexpr int Gk = decltype(gc)::value;
    Mfma<T>::run(fb[Gk][i / MB], fa[Gk][i % MB], acc[i / MB][i % MB]);
  };
  using G0 = std::integral_constant<int, 0>;
  using G1 = std::integral_constant<int, 1>;

  // Stage s of the stream. MODE 0: s = 0 (its Y loads were part of the prologue); 1: a
  // steady stage (Y loads of stage s + 2, X loads of stage s + 3); 2: s = S - 3 (Y loads
  // only); 3: s = S - 2 (no loads); 4: s = S - 1 (nothing follows). The second half of
  // modes 0 and 1, and the end of the prologue, issue exactly IDXL index DMAs (the next
  // offset's indices when cursor X has entered an offset, else dummies) before the X
  // loads, so the wait before the barriers of modes 0..2 is always L + IDXL (at most
  // one set of index DMAs older than the loads it waits for is then left in flight).
  auto stage = [&](Cursor& cx, Cursor& cy, int slot, auto modec) {
    constexpr int MODE = decltype(modec)::value;
    constexpr bool yload = MODE == 1 || MODE == 2, xload = MODE <= 1, next = MODE != 4;
    // first half: K-group 0 MFMAs, K-group 1 fragment reads, Y loads of stage s + 2
    wait_lgkm0();
    if constexpr (yload) {
      if (cy.kb == 0) {
        enter_offset(cy, YC{});
        wait_lgkm0();
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NM; ++i) {
      mma_one(G0{}, i);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int f = i * NF / NM; f < (i + 1) * NF / NM; ++f) frag_one(slot, G1{}, f);
      if constexpr (yload) {
        if (i >= NM - (L - LX)) issue(cy, LX + i - (NM - (L - LX)));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (yload) advance(cy);
    if constexpr (MODE <= 2) wait_vmcnt<L + IDXL>();
    else if constexpr (MODE == 3) wait_vmcnt<0>();
    if constexpr (next) raw_barrier();
    // second half: K-group 1 MFMAs, K-group 0 fragment reads of stage s + 1, X loads of
    // stage s + 3 (entering a new offset first: its sources, and the next offset's indices)
    wait_lgkm0();
    if constexpr (xload) {
      if (cx.kb == 0) {
        enter_offset(cx, XC{});
        if (cx.rest) {
          issue_idx(__builtin_ctz(cx.rest), (cx.ord + 1) & 1);
        } else {
#pragma unroll
          for (int u = 0; u < IDXL; ++u) lds_dma4(a.gidx + lane, idx_dummy);
        }
        wait_lgkm0();
      } else {
#pragma unroll
        for (int u = 0; u < IDXL; ++u) lds_dma4(a.gidx + lane, idx_dummy);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    const int nslot = (slot + 1) & (NS - 1);
#pragma unroll
    for (int i = 0; i < NM; ++i) {
      mma_one(G1{}, i);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (next) {
#pragma unroll
        for (int f = i * NF / NM; f < (i + 1) * NF / NM; ++f) frag_one(nslot, G0{}, f);
      }
      if constexpr (xload) {
        if (i >= NM - LX) issue(cx, i - (NM - LX));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (xload) advance(cx);
  };
  using M0 = std::integral_constant<int, 0>;
  using M1 = std::integral_constant<int, 1>;
  using M2 = std::integral_constant<int, 2>;
  using M3 = std::integral_constant<int, 3>;
  using M4 = std::integral_constant<int, 4>;

  if (S > 0) {  // S = taps * KB, KB >= 2
    Cursor cx, cy;
    start(cx);
    start(cy);
    // prologue: the first two offsets' indices; then stages 0..2 (those that exist),
    // entering the second offset on the way when KB < 3
    issue_idx(cx.k, 0);
    if (taps > 1) issue_idx(__builtin_ctz(cx.rest), 1);
    wait_vmcnt<0>();
    raw_barrier();
    enter_offset(cx, XC{});
    enter_offset(cy, YC{});
    bool x_entered = false;
#pragma unroll
    for (int st = 0; st < NS - 1; ++st) {
      if (st < S) {
#pragma unroll
        for (int u = 0; u < LX; ++u) issue(cx, u);
#pragma unroll
        for (int u = LX; u < L; ++u) issue(cy, u);
        // (stage 3 and later enter their offsets in the stage loop)
        if (advance(cx) && st + 1 < NS - 1 && st + 1 < S) {
          enter_offset(cx, XC{});
          x_entered = true;
        }
        if (advance(cy) && st + 1 < NS - 1 && st + 1 < S) enter_offset(cy, YC{});
      }
    }
    if (S >= 4) {
      // the offset after the one cursor X entered in the prologue (else dummies): the
      // steady-state rule, issued after the prologue's loads
      if (x_entered && cx.rest) {
        issue_idx(__builtin_ctz(cx.rest), (cx.ord + 1) & 1);
      } else {
#pragma unroll
        for (int u = 0; u < IDXL; ++u) lds_dma4(a.gidx + lane, idx_dummy);
      }
      wait_vmcnt<2 * L + IDXL>();
      raw_barrier();
#pragma unroll
      for (int i = 0; i < NF; ++i) frag_one(0, G0{}, i);

      stage(cx, cy, 0, M0{});
      int slot = 1;
      for (int s = 1; s + 3 < S; ++s) {
        stage(cx, cy, slot, M1{});
        slot = (slot + 1) & (NS - 1);
      }
      stage(cx, cy, slot, M2{});
      stage(cx, cy, (slot + 1) & (NS - 1), M3{});
      stage(cx, cy, (slot + 2) & (NS - 1), M4{});
    } else {
      // two or three stages: all of them are in the ring
      wait_vmcnt<0>();
      raw_barrier();
#pragma unroll
      for (int i = 0; i < NF; ++i) frag_one(0, G0{}, i);
      for (int s = 0; s + 1 < S; ++s) stage(cx, cy, s, M3{});
      stage(cx, cy, S - 1, M4{});
    }
  }

  // epilogue: each wave stages its (MB * 32) x (NB * 32) block
  wait_vmcnt<0>();
  __syncthreads();
  const bool has_bias = a.bias != nullptr;
  constexpr int ES = static_cast<int>(sizeof(T));
  constexpr int EPC = 16 / ES;          // elements per 16-byte chunk
  constexpr int ROWB = NB * 32 * ES;    // staged row bytes
  constexpr int CPR = ROWB / 16;        // 16-byte chunks per staged row
  using Quad = std::conditional_t<ES == 2, uint2, u32x4>;  // a lane's 4 consecutive channels
  char* stg = smem + wave * (MB * 32 * ROWB);
  const int cb = n0 + wn * NB * 32;
  // convert (bias, the activation) and stage; the activation is chosen once, outside
  // the element loops
  auto stage_acc = [&](auto silu) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int j0 = nb * 32 + 8 * q + 4 * (lane >> 5);
        float b[4];
        {
          T bt[4];
          __builtin_memcpy(bt, s_bias + ((cb - n0) + j0) * sizeof(T), sizeof(bt));
#pragma unroll
          for (int e = 0; e < 4; ++e) b[e] = has_bias ? to_f32(bt[e]) : 0.0f;
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const int row = mb * 32 + (lane & 31);
          T h[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float x = acc[nb][mb][4 * q + e] + b[e];
            if constexpr (decltype(silu)::value) x = silu_f32(x);
            h[e] = static_cast<T>(x);
          }
          Quad packed;
          __builtin_memcpy(&packed, h, sizeof(Quad));
          const int byte = j0 * ES;  // 16-byte chunk byte / 16, offset byte % 16 inside it
          *reinterpret_cast<Quad*>(stg + row * ROWB + (((byte >> 4) ^ (row & (CPR - 1))) << 4) + (byte & 15)) = packed;
        }
      }
    }
  };
  if (a.act == HI3D_ACT_SILU) stage_acc(std::true_type{});
  else stage_acc(std::false_type{});
  wait_lgkm0();
  const int64_t out_row_bytes = static_cast<int64_t>(a.cout) * ES;
#pragma unroll 4
  for (int i = 0; i < MB * 32 * CPR / 64; ++i) {
    const int row = lane / CPR + (64 / CPR) * i;  // within this wave's MB * 32 rows
    const int chunk = lane % CPR;
    const int tr = wm * (MB * 32) + row;
    const int64_t pt = tile * SUB + tr / kTileRows;
    if (pt >= a.ntiles) continue;
    const int32_t orow = reinterpret_cast<const int32_t*>(rows_lds)[tr];
    if (orow < 0 || orow >= a.n_out) continue;
    u32x4 v = *reinterpret_cast<const u32x4*>(stg + row * ROWB + ((chunk ^ (row & (CPR - 1))) << 4));
    const int64_t off = static_cast<int64_t>(orow) * out_row_bytes + static_cast<int64_t>(cb + chunk * EPC) * ES;
    if (a.residual != nullptr) {
      v = add_chunk<T>(v, *reinterpret_cast<const u32x4*>(a.residual + off));
    }
    *reinterpret_cast<u32x4*>(a.out + off) = v;
  }
}

template <typename T, int BN, int NW, int BM = RingShape<BN, NW>::BM>
int launch_ring(const ConvArgs& base, hipStream_t stream) {
  ConvArgs a = base;
  a.ny = a.cout / BN;
  const int64_t blocks = ceil_div(a.ntiles, RingShape<BN, NW, BM>::SUB) * a.ny;
  if (blocks == 0) return HI3D_OK;
  HI3D_REQUIRE(blocks < (int64_t(1) << 31), "too many tiles");
  hipLaunchKernelGGL((conv_ring_kernel<T, BN, NW, BM>), dim3(static_cast<unsigned>(blocks)), dim3(NW * 64), 0, stream, a);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

// ------------------------------------------------------ fp32 16-row block kernel --
// fp32 rows of 64 channels into CO-channel output slices, for sets too small to fill
// the chip with 128-row tiles. A workgroup takes 16 NW plan rows and each wave one
// 16-row block, whose 16 x CO output block it accumulates in CO / 4 registers with
// v_mfma_f32_16x16x4f32: the weights are the A operand and the gathered rows B, so a
// lane ends with four consecutive output channels of its own row. A wave runs the
// MFMAs of only the offsets present in its 16 rows (1.15 products per present pair on
// the 45k-voxel C64 shell, against 1.59 for a 128-row tile's union); the workgroup
// walks the union of its blocks' offsets in step, so that each offset's weight slice
// (CO x 256 bytes) is loaded into LDS once (NSLOT slices in flight), while each wave
// gathers its rows straight into registers one offset ahead. On that shell: 70 us for
// eight waves, two slices and 32 channels, against 110 us for the 128-row ring tile
// (four waves over 64 channels 72 us, three slices 78-100 us, 16 channels 88 us).
// Every workgroup is resident from the start, and per-wave timestamps put each CU's
// end in proportion to the offsets its waves run (correlation 0.97, 0.36 us per
// wave-offset); dealing the tiles or a workgroup's blocks in other orders (across the
// XCDs, heaviest first, heavy with light on one SIMD) left the time unchanged.
//
// K order: lane (i, h) = (lane % 16, lane / 16) loads 16 bytes of its row, channels
// 16 s + 4 h .. + 3, and MFMA j of step s takes channel 16 s + 4 h + j from both
// operands, so the 16 (s, j) MFMAs cover each channel once.
constexpr int kBlockRows = 16;
constexpr int kBlockCin = 64;
constexpr int kBlockCout = 64;

template <int NW, int NSLOT, int CO>
__global__ __launch_bounds__(NW * 64) void conv_block_f32_kernel(ConvArgs a) {
  constexpr int R = kBlockRows * NW;                // plan rows per workgroup
  constexpr int SLICE = CO * kBlockCin * 4;         // one offset's weights for the CO output channels, bytes
  constexpr int NCB = CO / 16;                      // 16-channel output blocks
  constexpr int DW = SLICE / (1024 * NW);           // 1 KB weight DMAs per wave and offset
  constexpr int KV = kMaxPipelinedKvol;
  static_assert(DW * NW * 1024 == SLICE && kTileRows % R == 0 && (CO == 16 || CO == 32 || CO == 64), "shape");
  static_assert(NSLOT == 2 || NSLOT == 3, "two or three weight slices in flight");
  // weight slices (row c = output channel, 256 bytes; 16-byte chunk q of row c at
  // position q ^ (c % 16)), then the blocks' gather rows [k][R] (-1: absent), then masks
  __shared__ __attribute__((aligned(16))) char smem[NSLOT * SLICE + KV * R * 4 + NW * 4];
  int32_t* const gl = reinterpret_cast<int32_t*>(smem + NSLOT * SLICE);
  uint32_t* const smask = reinterpret_cast<uint32_t*>(gl + KV * R);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 15, h = lane >> 4;
  const int64_t item = xcd_remap(blockIdx.x, static_cast<int64_t>(gridDim.x));
  const int64_t tile = item / a.ny;
  const int n0 = static_cast<int>(item - tile * a.ny) * CO;
  const int kvol = a.kvol;
  const uint64_t n_in = static_cast<uint64_t>(a.n_in);
  const int brow = wave * kBlockRows + i;  // this lane's row in the workgroup
  const int64_t p = tile * R + brow;       // its plan row (< ntiles * 128: R divides 128)
  const int32_t orow = a.rows[p];
  const int32_t* gsrc = a.gidx + (p / kTileRows) * kvol * kTileRows + (p % kTileRows);

  // the block's gather rows into LDS and its offset mask
  // (all loads issued before the first use: offsets past kvol reread offset 0)
  int32_t g[KV];
#pragma unroll
  for (int k = 0; k < KV; ++k) g[k] = gsrc[(k < kvol ? k : 0) * kTileRows];
  uint32_t wmask = 0;
#pragma unroll
  for (int k = 0; k < KV; ++k) {
    const bool ok = k < kvol && static_cast<uint64_t>(static_cast<uint32_t>(g[k])) < n_in;
    if (__builtin_amdgcn_ballot_w64(ok) != 0) wmask |= 1u << k;
    if (h == 0) gl[k * R + brow] = ok ? g[k] : -1;
  }
  if (lane == 0) smask[wave] = wmask;
  __syncthreads();
  uint32_t uni = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) uni |= smask[w];
  uni = __builtin_amdgcn_readfirstlane(uni);
  const int n = __popc(uni);

  // DMA u of this wave fills slice bytes [1024 m, +1024), m = wave + NW u: row
  // c = 4 m + lane / 16, position lane % 16, i.e. logical chunk (lane % 16) ^ (c % 16)
  auto issue_w = [&](int k, int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < DW; ++u) {
      const int m = wave + NW * u;
      const int c = 4 * m + (lane >> 4);
      const int q = (lane & 15) ^ (c & 15);
      lds_dma16(a.weight + (static_cast<int64_t>(n0 + c) * kvol + k) * (kBlockCin * 4) + q * 16,
                smem + slot * SLICE + m * 1024);
    }
  };
  // gathered rows through global (not flat) loads, which LDS waits do not cover
  using GRow = const __attribute__((address_space(1))) f32x4;
  const char* const zrow = reinterpret_cast<const char*>(g_zero_row) + h * 16;
  auto issue_x = [&](int k, f32x4 (&x)[4]) __attribute__((always_inline)) {
    const int32_t gk = gl[k * R + brow];
    const char* src = gk >= 0 ? a.in + static_cast<int64_t>(gk) * (kBlockCin * 4) + h * 16 : zrow;
#pragma unroll
    for (int s = 0; s < 4; ++s) x[s] = *(GRow*)(src + 64 * s);
  };
  f32x4 acc[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) acc[cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  auto compute = [&](int slot, const f32x4 (&x)[4]) __attribute__((always_inline)) {
    const char* sb = smem + slot * SLICE + i * 256;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      f32x4 wf[NCB];
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb)
        wf[cb] = *reinterpret_cast<const f32x4*>(sb + cb * (16 * 256) + (((4 * s + h) ^ i) << 4));
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) acc[cb] = __builtin_amdgcn_mfma_f32_16x16x4f32(wf[cb][j], x[s][j], acc[cb], 0, 0, 0);
    }
  };

  if (n > 0) {
    // offsets of ordinals ord, ord + 1, ord + 2 (the later ones meaningless past n)
    uint32_t rest = uni;
    auto pop = [&]() __attribute__((always_inline)) {
      const int k = rest ? __builtin_ctz(rest) : 0;
      rest &= rest - 1u;
      return k;
    };
    int kc = pop(), kx = pop(), kw = pop();
    f32x4 xa[4], xb[4];
    // prologue, in issue order: W(0), X(0), then W(1) with three slices
    issue_w(kc, 0);
    issue_x(kc, xa);
    if constexpr (NSLOT == 3) {
      if (n > 1) issue_w(kx, 1);
    }
    int slot = 0;
    // iteration ord: wait for W(ord) and X(ord) (with three slices W(ord + 1), issued
    // after them, may stay in flight), so that after the barrier every wave's share of
    // slice ord is in LDS and slice ord - 1 is no longer read; then X(ord + 1) and the
    // next slice, then the MFMAs of ord when this block has the offset
    auto body = [&](int ord, const f32x4 (&xc)[4], f32x4 (&xn)[4]) __attribute__((always_inline)) {
      if (NSLOT == 3 && ord + 1 < n) wait_vmcnt<DW>();
      else wait_vmcnt<0>();
      raw_barrier();
      if (ord + 1 < n) issue_x(kx, xn);
      if constexpr (NSLOT == 3) {
        if (ord + 2 < n) issue_w(kw, slot == 0 ? 2 : slot - 1);
      } else {
        if (ord + 1 < n) issue_w(kx, slot ^ 1);
      }
      if ((wmask >> kc) & 1u) compute(slot, xc);
      slot = NSLOT == 3 ? (slot == 2 ? 0 : slot + 1) : (slot ^ 1);
      kc = kx;
      kx = kw;
      kw = pop();
    };
    for (int ord = 0; ord < n; ord += 2) {
      body(ord, xa, xb);
      if (ord + 1 < n) body(ord + 1, xb, xa);
    }
  }

  // epilogue: lane (i, h) holds output channels n0 + 16 cb + 4 h .. + 3 of its row
  if (orow < 0 || orow >= a.n_out) return;
  const float* bias = static_cast<const float*>(a.bias);
  const int64_t obase = static_cast<int64_t>(orow) * a.cout * 4;
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const int col = n0 + 16 * cb + 4 * h;
    f32x4 v = acc[cb];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float x = v[e] + (bias != nullptr ? bias[col + e] : 0.0f);
      if (a.act == HI3D_ACT_SILU) x = silu_f32(x);
      v[e] = x;
    }
    const int64_t off = obase + col * 4;
    if (a.residual != nullptr) v += *reinterpret_cast<const f32x4*>(a.residual + off);
    *reinterpret_cast<f32x4*>(a.out + off) = v;
  }
}

template <int NW, int NSLOT, int CO>
int launch_block_f32(const ConvArgs& base, hipStream_t stream) {
  ConvArgs a = base;
  a.ny = a.cout / CO;
  const int64_t blocks = ceil_div(a.n_out, kBlockRows * NW) * a.ny;
  if (blocks == 0) return HI3D_OK;
  HI3D_REQUIRE(blocks < (int64_t(1) << 31), "too many tiles");
  hipLaunchKernelGGL((conv_block_f32_kernel<NW, NSLOT, CO>), dim3(static_cast<unsigned>(blocks)), dim3(NW * 64), 0, stream,
                     a);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

// ------------------------------------------------------ wide-step ring kernel --
// The ring kernel's scheme with 128-byte K steps: each gathered row is fetched as one
// 128-byte request per stage instead of two 64-byte ones, halving the gather requests
// per flop (L2-resident gathers: ~24 TB/s with 128-byte rows against ~15 TB/s with
// 64-byte rows). Stages of (BM + BN) x 128 bytes = 48 KB sit in a 3-deep ring.
//  * Tile: BN = 128 takes BM = 256 rows, BN = 256 takes BM = 128 rows; NW waves form a
//    BM / 64 x NW / (BM / 64) grid, each owning 64 rows x its channels as 2 x NB blocks
//    of 32x32x16 MFMAs, four K-groups of 16 elements per stage.
//  * Loads: per wave L = (BM + BN) / (8 NW) direct-to-LDS 16-byte loads per stage
//    (8 lanes per 128-byte row), all for stage s + 2, issued in K-groups 0..2 of stage
//    s, L / 3 after the last MFMAs of each. Stage s + 2 reuses the slot of stage s - 1,
//    whose last fragment reads precede the barrier of stage s - 1.
//  * One barrier per stage, before K-group 3 (whose fragment reads are stage s + 1's
//    K-group 0): the wait before it leaves exactly stage s + 2's L loads in flight,
//    plus the next offset's index load when one was issued in stage s.
//  * Rows use the 128-byte XOR swizzle (chunk c of row r at c ^ ((r >> 1) & 7)), so the
//    fragment reads are conflict-free; gather indices and the epilogue follow the ring
//    kernel.
template <int BN, int NW>
struct WideShape {
  static constexpr int BM = BN == 128 ? 256 : 128;
  static constexpr int WM = BM / 64;         // waves across rows (64 rows each)
  static constexpr int WN = NW / WM;         // waves across channels
  static constexpr int NB = BN / WN / 32;    // channel blocks per wave
  static constexpr int SUB = BM / kTileRows;
  static constexpr int LA = BM / (8 * NW);   // gathered-row loads per wave and stage
  static constexpr int LB = BN / (8 * NW);   // weight-row loads per wave and stage
  static constexpr int L = LA + LB;
  static constexpr int STAGE_A = BM * 128;
  static constexpr int STAGE = STAGE_A + BN * 128;
  static constexpr int IDX = BM * 4;
};
constexpr int kWideDepth = 3;

__device__ __forceinline__ int wide_off(int row, int chunk) { return row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4); }

template <typename T, int BN, int NW, bool K1, bool kLN = false>
__global__ __launch_bounds__(NW * 64, 1) void conv_wide_kernel(ConvArgs a) {
  using Sh = WideShape<BN, NW>;
  constexpr int NS = kWideDepth, BM = Sh::BM, LA = Sh::LA, LB = Sh::LB, SUB = Sh::SUB, L = Sh::L;
  constexpr int STAGE = Sh::STAGE, STAGE_A = Sh::STAGE_A, IDX = Sh::IDX;
  constexpr int MB = 2, NB = Sh::NB, NF = MB + NB, NM = MB * NB, KG = 4, LG = L / (KG - 1);
  static_assert(STAGE == 49152 && LG * (KG - 1) == L && LG <= NM && LA * 8 * NW == BM, "stage shape");
  static_assert(sizeof(T) == 2, "16-bit elements (the epilogue packs four channels into 8 bytes)");
  static_assert(BM * BN * 2 <= NS * STAGE, "output tile must fit the ring");
  // gather-index ring: two slots (one offset ahead), or with K1 (128-byte rows, one K
  // stage per offset) four, two offsets ahead, so that a request has a whole stage to land
  constexpr int ISLOTS = K1 ? 4 : 2;
  constexpr int AHEAD = K1 ? 2 : 1;  // offsets between an index request and its use
  constexpr int kBiasDwords = BN * static_cast<int>(sizeof(T)) / 4;
  constexpr int kBiasBytes = (kBiasDwords + 63) / 64 * 256;
  // one LDS array (a second one makes the compiler wait for every direct-to-LDS load
  // before each LDS read); the tile's bias sits at its end
  __shared__ __attribute__((aligned(16))) char smem[NS * STAGE + (ISLOTS + 1) * IDX + 256 + kBiasBytes];
  char* const s_bias = smem + (NS * STAGE + (ISLOTS + 1) * IDX + 256);
  char* const idx_ring = smem + NS * STAGE;
  char* const rows_lds = idx_ring + ISLOTS * IDX;  // the tile's output rows
  char* const idx_dummy = rows_lds + IDX;     // target of the index DMA of stages entering no offset

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % Sh::WM, wn = wave / Sh::WM;
  const int64_t item = xcd_remap(blockIdx.x, static_cast<int64_t>(gridDim.x));
  const int64_t tile = item / a.ny;
  const int n0 = static_cast<int>(item - tile * a.ny) * BN;
  // the tile's bias reaches LDS by 4-byte DMAs before any stage is requested: the
  // oldest loads, so the stage loop's constant waits still hold, and no register waits
  // on them (the epilogue reads it after its wait for every load)
  if (a.bias != nullptr && wave < (kBiasDwords + 63) / 64) {
    const int d = wave * 64 + lane;
    lds_dma4(static_cast<const char*>(a.bias) + static_cast<int64_t>(n0) * sizeof(T) + 4 * (d < kBiasDwords ? d : kBiasDwords - 1),
             s_bias + wave * 256);
  }
  const int kvol = a.kvol;
  uint32_t mask = 0;
#pragma unroll
  for (int h = 0; h < SUB; ++h) {
    const int64_t pt = tile * SUB + h;
    if (pt < a.ntiles) mask |= a.tile_mask[pt];
  }
  mask &= (1u << kvol) - 1u;
  const int rb = a.cin * static_cast<int>(sizeof(T));
  const int KB = rb >> 7;
  const int taps = __popc(mask);
  const int S = taps * KB;
  const uint64_t n_in = static_cast<uint64_t>(a.n_in);

  // load j of this wave covers rows (wave + NW j) * 8 + lane / 8 at physical chunk
  // lane % 8, i.e. logical chunk coff / 16 (the swizzle repeats every 16 rows)
  const int r0 = wave * 8 + (lane >> 3);
  const int coff = ((lane & 7) ^ ((r0 >> 1) & 7)) * 16;
  const char* wrow[LB];
#pragma unroll
  for (int j = 0; j < LB; ++j)
    wrow[j] = a.weight + static_cast<int64_t>(n0 + r0 + 8 * NW * j) * kvol * rb + coff;
  const char* const zrow = reinterpret_cast<const char*>(g_zero_row) + coff;

  // gather indices of offset k into slot `slot`: load `wave` of BM / 64 covers rows
  // 64 wave .. +63 (waves beyond BM / 64 repeat the last one)
  auto issue_idx = [&](int k, int slot) {
    const int i = wave < BM / 64 ? wave : BM / 64 - 1;
    int64_t pt = tile * SUB + (i >> 1);
    if (pt >= a.ntiles) pt = a.ntiles - 1;
    lds_dma4(a.gidx + (pt * kvol + k) * kTileRows + (i & 1) * 64 + lane, idx_ring + slot * IDX + i * 256);
  };

  {  // the tile's output rows reach LDS at the start (complete by the first wait)
    const int i = wave < BM / 64 ? wave : BM / 64 - 1;
    int64_t pt = tile * SUB + (i >> 1);
    if (pt >= a.ntiles) pt = a.ntiles - 1;
    lds_dma4(a.rows + pt * kTileRows + (i & 1) * 64 + lane, rows_lds + i * 256);
  }

  uint32_t rest;  // offsets after the current one of the load cursor
  int ck, ckb, cord;
  const char* src[LA];
  auto enter_offset = [&]() {
    const int32_t* gi = reinterpret_cast<const int32_t*>(idx_ring + (cord & (ISLOTS - 1)) * IDX);
    int32_t g[LA];
#pragma unroll
    for (int j = 0; j < LA; ++j) g[j] = gi[r0 + 8 * NW * j];
#pragma unroll
    for (int j = 0; j < LA; ++j) src[j] = gather_src(a.in, g[j], n_in, rb, coff, zrow);
  };
  // offset whose indices are requested on entering an offset: the next one, or with one
  // K stage per offset the one after it (the current one again past the last)
  auto ahead_offset = [&]() {
    const uint32_t r = K1 ? rest & (rest - 1u) : rest;
    return r ? __builtin_ctz(r) : ck;
  };
  auto advance = [&]() {
    if (++ckb == KB) {
      ckb = 0;
      ck = rest ? __builtin_ctz(rest) : ck;
      rest &= rest - 1u;
      ++cord;
    }
  };
  auto issue_load = [&](int slot, int u) {  // u = 0..L-1: LA gathered, then LB weight loads
    char* st = smem + slot * STAGE;
    if (u < LA)
      lds_dma16(src[u] + ckb * 128, st + (wave + NW * u) * 1024);
    else
      lds_dma16(wrow[u - LA] + ck * rb + ckb * 128, st + STAGE_A + (wave + NW * (u - LA)) * 1024);
  };

  f32x16 acc[NB][MB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[nb][mb][v] = 0.0f;
  u32x4 fa[2][MB], fb[2][NB];
  auto frag_one = [&](int slot, auto gc, int i) {  // K-group G of the stage in `slot`
    constexpr int G = decltype(gc)::value;
    const char* st = smem + slot * STAGE;
    const int c = 2 * G + (lane >> 5);
    if (i < NB)
      fb[G & 1][i] = *reinterpret_cast<const u32x4*>(st + STAGE_A + wide_off(wn * NB * 32 + i * 32 + (lane & 31), c));
    else
      fa[G & 1][i - NB] = *reinterpret_cast<const u32x4*>(st + wide_off(wm * 64 + (i - NB) * 32 + (lane & 31), c));
  };
  auto mma_one = [&](auto gc, int i) {  // i = nb * MB + mb
    constexpr int G = decltype(gc)::value;
    Mfma<T>::run(fb[G & 1][i / MB], fa[G & 1][i % MB], acc[i / MB][i % MB]);
  };
  using G0 = std::integral_constant<int, 0>;
  using G1 = std::integral_constant<int, 1>;
  using G2 = std::integral_constant<int, 2>;
  using G3 = std::integral_constant<int, 3>;

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  // Stage s of the stream in ring slot SL = s % 3. MODE 0: a steady stage (loads stage
  // s + 2, stage s + 1 follows); 1: stage S - 2 (no loads); 2: stage S - 1 (no loads,
  // nothing follows). A steady stage issues exactly one index DMA (the next offset's
  // indices when stage s + 2 begins an offset, else a dummy) and then its L loads, so
  // the wait before its barrier is always L + 1.
  auto stage = [&](int SL, auto modec) {
    constexpr int MODE = decltype(modec)::value;
    const int LS = SL == 0 ? NS - 1 : SL - 1, NSL = SL == NS - 1 ? 0 : SL + 1;
    if constexpr (MODE == 0) {
      if (ckb == 0) {
        wait_lgkm0();
        enter_offset();
        issue_idx(ahead_offset(), (cord + AHEAD) & (ISLOTS - 1));
      } else {
        lds_dma4(a.gidx + lane, idx_dummy);
      }
    }
    auto group = [&](auto gc) {
      constexpr int G = decltype(gc)::value;
      wait_lgkm0();
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < NM; ++i) {
        mma_one(gc, i);
        __builtin_amdgcn_sched_barrier(0);
        if (i < NF) {
          if constexpr (G < KG - 1)
            frag_one(SL, std::integral_constant<int, G + 1>{}, i);
          else if constexpr (MODE != 2)
            frag_one(NSL, G0{}, i);
        }
        if constexpr (G < KG - 1 && MODE == 0) {
          if (i >= NM - LG) issue_load(LS, G * LG + i - (NM - LG));
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    group(G0{});
    group(G1{});
    group(G2{});
    if constexpr (MODE == 0) {
      advance();
      wait_vmcnt<L + 1>();
      raw_barrier();
    } else if constexpr (MODE == 1) {
      wait_vmcnt<0>();
      raw_barrier();
    }
    group(G3{});
  };

  if (S > 0) {  // S = taps * KB (1 only for one tap of a 128-byte row)
    ck = mask ? __builtin_ctz(mask) : 0;
    rest = mask & (mask - 1u);
    ckb = 0;
    cord = 0;
    issue_idx(ck, 0);
    if constexpr (K1) issue_idx(rest ? __builtin_ctz(rest) : ck, 1);
    wait_vmcnt<0>();
    raw_barrier();
    enter_offset();
    // prologue: the next offset's indices (offset 0's again without a successor), then
    // stages 0 and 1 (with S = 1, stage 1 rereads stage 0's rows into slot 1, unused;
    // the epilogue's wait retires it)
    issue_idx(ahead_offset(), AHEAD);
#pragma unroll
    for (int st = 0; st < NS - 1; ++st) {
#pragma unroll
      for (int u = 0; u < L; ++u) issue_load(st, u);
      advance();
      if (K1 && st == 0) {
        // stage 1 is the second offset's, whose indices came with the first's
        enter_offset();
        issue_idx(ahead_offset(), (cord + 2) & 3);
      }
    }
    // stage 0's loads land (with one K stage per offset also the third offset's
    // indices, requested before them; the fourth's may stay in flight)
    if constexpr (K1) wait_vmcnt<L + 1>();
    else wait_vmcnt<L>();
    raw_barrier();
#pragma unroll
    for (int i = 0; i < NF; ++i) frag_one(0, G0{}, i);

    if (K1 && S == 1) {
      stage(0, I2{});
    } else {
      int slot = 0;
      for (int s = 0; s + 2 < S; ++s) {
        stage(slot, I0{});
        slot = slot == NS - 1 ? 0 : slot + 1;
      }
      // the last two stages, S - 2 and S - 1
      stage(slot, I1{});
      stage(slot == NS - 1 ? 0 : slot + 1, I2{});
    }
  }

  // epilogue: each wave stages its 64 x (NB * 32) block
  wait_vmcnt<0>();
  __syncthreads();
  const bool has_bias = a.bias != nullptr;
  constexpr int ROWB = NB * 64, CPR = NB * 4;
  char* stg = smem + wave * (64 * ROWB);
  const int cb = n0 + wn * NB * 32;
  const int64_t out_row_bytes = static_cast<int64_t>(a.cout) * sizeof(T);
  // chunk i of this lane: row lane / CPR + (64 / CPR) i of the wave's rows, 16-byte chunk
  // lane % CPR of its channels; false for rows past the plan or without an output row
  // the output rows of this lane's chunks, all read from LDS at once (one wait, not one
  // per chunk)
  int32_t orow[CPR];
#pragma unroll
  for (int i = 0; i < CPR; ++i) {
    const int tr = wm * 64 + lane / CPR + (64 / CPR) * i;
    const int64_t pt = tile * SUB + tr / kTileRows;
    orow[i] = pt < a.ntiles ? reinterpret_cast<const int32_t*>(rows_lds)[tr] : -1;
  }
  auto chunk_ok = [&](int i) { return orow[i] >= 0 && orow[i] < a.n_out; };
  auto chunk_off = [&](int i) {
    return static_cast<int64_t>(orow[i]) * out_row_bytes + static_cast<int64_t>(cb + (lane % CPR) * 8) * sizeof(T);
  };
  // the residual's chunks are requested before the accumulators are converted and
  // staged, so their latency overlaps that work instead of each group of stores
  u32x4 res[CPR];
  if (a.residual != nullptr) {
#pragma unroll
    for (int i = 0; i < CPR; ++i) res[i] = *reinterpret_cast<const u32x4*>(a.residual + (chunk_ok(i) ? chunk_off(i) : 0));
  }
  // convert (bias, the activation) and stage; the activation is chosen once, outside
  // the element loops
  auto stage_acc = [&](auto silu) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int j0 = nb * 32 + 8 * q + 4 * (lane >> 5);
        float b[4];
        {
          T bt[4];
          __builtin_memcpy(bt, s_bias + ((cb - n0) + j0) * sizeof(T), sizeof(bt));
#pragma unroll
          for (int e = 0; e < 4; ++e) b[e] = has_bias ? to_f32(bt[e]) : 0.0f;
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const int row = mb * 32 + (lane & 31);
          T h[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float x = acc[nb][mb][4 * q + e] + b[e];
            if constexpr (decltype(silu)::value) x = silu_f32(x);
            h[e] = static_cast<T>(x);
          }
          uint2 packed;
          __builtin_memcpy(&packed, h, 8);
          *reinterpret_cast<uint2*>(stg + row * ROWB + (((j0 >> 3) ^ (row & (CPR - 1))) << 4) + (j0 & 4) * 2) = packed;
        }
      }
    }
  };
  if (a.act == HI3D_ACT_SILU) stage_acc(std::true_type{});
  else stage_acc(std::false_type{});
  wait_lgkm0();
  if constexpr (kLN) {
    // The res block's second norm on whole output rows (cout == BN == 128): each row's
    // 16 chunks sit in the staged blocks of waves (row / 64) (chunks 0..7) and
    // (row / 64) + 4 (chunks 8..15). Eight lanes per row, lane g holding chunks g and
    // g + 8: the lanes, chunks, summation order and reduction partners of ln_kernel<8, 2>
    // (the LayerNorm of 128-channel rows), so the result is bitwise the convolution
    // followed by that kernel.
#pragma clang fp contract(off)
    static_assert(BN == 128 && NB == 2 && Sh::WM == 4 && NW == 8, "the row norm takes whole 128-channel rows");
    __syncthreads();
    const _Float16* scale = static_cast<const _Float16*>(a.ln_scale);
    const _Float16* shift = static_cast<const _Float16*>(a.ln_shift);
    const int g = lane & 7;
    const float c = static_cast<float>(BN);
    // the four passes are unrolled so that their independent chains (LDS reads, sums,
    // lane moves, the square root and the SiLU) overlap; lane moves by DPP (the same
    // partners as ln_kernel's shuffles)
#pragma unroll
    for (int pass = 0; pass < BM / (NW * 8); ++pass) {
      const int tr = pass * (NW * 8) + wave * 8 + (lane >> 3);  // tile row
      const int64_t pt = tile * SUB + tr / kTileRows;
      const int32_t lrow = pt < a.ntiles ? reinterpret_cast<const int32_t*>(rows_lds)[tr] : -1;
      const bool live = lrow >= 0 && lrow < a.n_out;
      const int wr = tr & 63;
      float v[2][8];
      float sum = 0.0f;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const f16x8 h = *reinterpret_cast<const f16x8*>(smem + ((tr >> 6) + 4 * i) * (64 * ROWB) + wr * ROWB +
                                                        ((g ^ (wr & (CPR - 1))) << 4));
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          v[i][e] = static_cast<float>(h[e]);
          sum += v[i][e];
        }
      }
      sum += dpp_xor4(sum);
      sum += dpp_xor2(sum);
      sum += dpp_xor1(sum);
      const float mean = sum / c;
      float sq = 0.0f;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = v[i][e] - mean;
          sq += d * d;
        }
      sq += dpp_xor4(sq);
      sq += dpp_xor2(sq);
      sq += dpp_xor1(sq);
      const float inv = 1.0f / sqrtf(sq / c + a.ln_eps);
      int b = live ? a.ln_coords[static_cast<int64_t>(lrow) * 4] : 0;
      b = b < 0 ? 0 : (b >= a.ln_batches ? a.ln_batches - 1 : b);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int ch = g + 8 * i;
        f16x8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = static_cast<_Float16>(f32_rounded((v[i][e] - mean) * inv));
        o = modulate8(o, *reinterpret_cast<const f16x8*>(scale + b * BN + ch * 8),
                      *reinterpret_cast<const f16x8*>(shift + b * BN + ch * 8));
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = silu_h(o[e]);
        if (live) *reinterpret_cast<f16x8*>(a.out + (static_cast<int64_t>(lrow) * BN + ch * 8) * 2) = o;
      }
    }
    return;
  }
  // every staged chunk is read before the first store (one LDS wait)
  u32x4 v[CPR];
#pragma unroll
  for (int i = 0; i < CPR; ++i) {
    const int row = lane / CPR + (64 / CPR) * i;  // 0..63 within this wave's rows
    v[i] = *reinterpret_cast<const u32x4*>(stg + row * ROWB + (((lane % CPR) ^ (row & (CPR - 1))) << 4));
  }
#pragma unroll
  for (int i = 0; i < CPR; ++i) {
    if (a.residual != nullptr) v[i] = add_chunk<T>(v[i], res[i]);
    if (chunk_ok(i)) *reinterpret_cast<u32x4*>(a.out + chunk_off(i)) = v[i];
  }
}

template <typename T, int BN, int NW, bool K1 = false, bool kLN = false>
int launch_wide(const ConvArgs& base, hipStream_t stream) {
  // the one-stage form (K1) takes 128-byte rows and the other form longer ones
  HI3D_REQUIRE(K1 == (base.cin * static_cast<int>(sizeof(T)) == 128), "wide kernel: row length and form disagree");
  ConvArgs a = base;
  a.ny = a.cout / BN;
  const int64_t blocks = ceil_div(a.ntiles, WideShape<BN, NW>::SUB) * a.ny;
  if (blocks == 0) return HI3D_OK;
  HI3D_REQUIRE(blocks < (int64_t(1) << 31), "too many tiles");
  hipLaunchKernelGGL((conv_wide_kernel<T, BN, NW, K1, kLN>), dim3(static_cast<unsigned>(blocks)), dim3(NW * 64), 0,
                     stream, a);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

// ------------------------------------------- 256 x 256 two-slot wide kernel --
// The wide kernel's 128-byte K steps at the 256 x 256 tile of the ring kernel: each
// gathered and weight row moves as one 128-byte request per stage (L2-resident gathers
// of 128-byte rows run ~1.6x the rate of 64-byte ones), at the ring kernel's gathered
// bytes per flop. A stage is (256 + 256) x 128 bytes = 64 KB, so the ring holds two.
//  * Tile: 256 output rows (two plan tiles, masks ORed) x 256 channels; 8 waves in a
//    4 x 2 grid, each 64 rows x 128 channels as 4 x 2 blocks of 32x32x16 MFMAs (weights
//    first), four K-groups of 16 elements per stage.
//  * Stage s: K-groups 0..2 (fragment reads of K-groups 1..3 of s, from its slot); a
//    wait for every outstanding load (those of stage s + 1, issued in K-group 3 of stage
//    s - 1) and the barrier; K-group 3, whose fragment reads are stage s + 1's K-group
//    0 and during which the wave issues its 8 loads of stage s + 2 (one after each
//    MFMA) into the slot of stage s, free after the barrier. A stage's loads thus have
//    K-group 3 of one stage and K-groups 0..2 of the next (~1,500 MFMA cycles per SIMD)
//    to land.
//  * Gather indices as in the other kernels: a two-slot ring, the next offset's 256
//    indices issued when the load cursor enters an offset (one index DMA per stage,
//    a dummy otherwise, so the waits stay exact: before each barrier nothing is in
//    flight but stage s + 1's loads and that DMA).
//  * Rows use the 128-byte XOR swizzle; the epilogue stages the fp16 tile over both
//    slots and writes 16-byte row chunks (bias, SiLU, residual as in the ring kernel).
constexpr int kW2Stage = 65536, kW2StageA = 32768, kW2Idx = 1024;

template <typename T>
__global__ __launch_bounds__(512, 1) void conv_wide2_kernel(ConvArgs a) {
  constexpr int BM = 256, BN = 256, NW = 8, WM = 4, NS = 2, SUB = BM / kTileRows;
  constexpr int MB = 2, NB = 4, NF = MB + NB, NM = MB * NB, LA = 4, LB = 4, L = LA + LB;
  static_assert(sizeof(T) == 2, "16-bit elements");
  static_assert(BM * BN * 2 <= NS * kW2Stage && LA * 8 * NW == BM && LB * 8 * NW == BN && L == NM, "shape");
  constexpr int kBiasDwords = BN * static_cast<int>(sizeof(T)) / 4;
  constexpr int kBiasBytes = (kBiasDwords + 63) / 64 * 256;
  // one LDS array (a second one makes the compiler wait for every direct-to-LDS load
  // before each LDS read); the tile's bias sits at its end
  __shared__ __attribute__((aligned(16))) char smem[NS * kW2Stage + 3 * kW2Idx + 256 + kBiasBytes];
  char* const s_bias = smem + (NS * kW2Stage + 3 * kW2Idx + 256);
  char* const idx_ring = smem + NS * kW2Stage;
  char* const rows_lds = idx_ring + 2 * kW2Idx;  // the tile's output rows
  char* const idx_dummy = rows_lds + kW2Idx;     // target of the index DMA of stages entering no offset

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Waves w and w + 4 share SIMD w % 4; they take row blocks w and w ^ 2, one from each
  // 128-row plan tile, so that an offset present in only one plan tile still gives
  // every SIMD one wave of MFMAs (a wave skips the offsets none of its rows has).
  const int wn = wave / WM, wm = (wave % WM) ^ (2 * wn);
  static_assert(WM == 4 && NW == 8, "crossed row blocks assume a 4 x 2 wave grid");
  const int64_t item = xcd_remap(blockIdx.x, static_cast<int64_t>(gridDim.x));
  const int64_t tile = item / a.ny;
  const int n0 = static_cast<int>(item - tile * a.ny) * BN;
  // the tile's bias reaches LDS by 4-byte DMAs before any stage is requested: the
  // oldest loads, so the stage loop's constant waits still hold, and no register waits
  // on them (the epilogue reads it after its wait for every load)
  if (a.bias != nullptr && wave < (kBiasDwords + 63) / 64) {
    const int d = wave * 64 + lane;
    lds_dma4(static_cast<const char*>(a.bias) + static_cast<int64_t>(n0) * sizeof(T) + 4 * (d < kBiasDwords ? d : kBiasDwords - 1),
             s_bias + wave * 256);
  }
  const int kvol = a.kvol;
  uint32_t mask = 0;
#pragma unroll
  for (int h = 0; h < SUB; ++h) {
    const int64_t pt = tile * SUB + h;
    if (pt < a.ntiles) mask |= a.tile_mask[pt];
  }
  mask &= (1u << kvol) - 1u;
  const int rb = a.cin * static_cast<int>(sizeof(T));
  const int KB = rb >> 7;
  const int taps = __popc(mask);
  const int S = taps * KB;
  const uint64_t n_in = static_cast<uint64_t>(a.n_in);

  // load j of this wave covers rows (wave + NW j) * 8 + lane / 8 at physical chunk
  // lane % 8, i.e. logical chunk coff / 16 (the swizzle repeats every 16 rows)
  const int r0 = wave * 8 + (lane >> 3);
  const int coff = ((lane & 7) ^ ((r0 >> 1) & 7)) * 16;
  const char* wrow[LB];
#pragma unroll
  for (int j = 0; j < LB; ++j)
    wrow[j] = a.weight + static_cast<int64_t>(n0 + r0 + 8 * NW * j) * kvol * rb + coff;
  const char* const zrow = reinterpret_cast<const char*>(g_zero_row) + coff;

  // gather indices of offset k into slot `slot`: wave w < 4 covers rows 64 w .. +63
  // (waves 4..7 repeat wave 3's load)
  auto issue_idx = [&](int k, int slot) {
    const int i = wave < BM / 64 ? wave : BM / 64 - 1;
    int64_t pt = tile * SUB + (i >> 1);
    if (pt >= a.ntiles) pt = a.ntiles - 1;
    lds_dma4(a.gidx + (pt * kvol + k) * kTileRows + (i & 1) * 64 + lane, idx_ring + slot * kW2Idx + i * 256);
  };
  {  // the tile's output rows reach LDS at the start (complete by the first wait)
    const int i = wave < BM / 64 ? wave : BM / 64 - 1;
    int64_t pt = tile * SUB + (i >> 1);
    if (pt >= a.ntiles) pt = a.ntiles - 1;
    lds_dma4(a.rows + pt * kTileRows + (i & 1) * 64 + lane, rows_lds + i * 256);
  }

  uint32_t rest;  // offsets after the current one of the load cursor
  int ck, ckb, cord;
  uint32_t pres = 0;  // bit o: the wave's 64 rows have the offset of ordinal o
  const char* src[LA];
  auto enter_offset = [&]() {
    const int32_t* gi = reinterpret_cast<const int32_t*>(idx_ring + (cord & 1) * kW2Idx);
    int32_t g[LA];
#pragma unroll
    for (int j = 0; j < LA; ++j) g[j] = gi[r0 + 8 * NW * j];
    const int32_t gw = gi[wm * 64 + lane];
#pragma unroll
    for (int j = 0; j < LA; ++j) src[j] = gather_src(a.in, g[j], n_in, rb, coff, zrow);
    if (__builtin_amdgcn_ballot_w64(static_cast<uint64_t>(static_cast<uint32_t>(gw)) < n_in) != 0) pres |= 1u << cord;
  };
  auto advance = [&]() {
    if (++ckb == KB) {
      ckb = 0;
      ck = rest ? __builtin_ctz(rest) : ck;
      rest &= rest - 1u;
      ++cord;
    }
  };
  auto issue_load = [&](int slot, int u) {  // u = 0..L-1: LA gathered, then LB weight loads
    char* st = smem + slot * kW2Stage;
    if (u < LA)
      lds_dma16(src[u] + ckb * 128, st + (wave + NW * u) * 1024);
    else
      lds_dma16(wrow[u - LA] + ck * rb + ckb * 128, st + kW2StageA + (wave + NW * (u - LA)) * 1024);
  };
  // the cursor's stage: enter its offset when it starts one (and fetch the next
  // offset's indices), else one dummy index DMA
  auto cursor_indices = [&]() {
    if (ckb == 0) {
      wait_lgkm0();
      enter_offset();
      issue_idx(rest ? __builtin_ctz(rest) : ck, (cord + 1) & 1);
    } else {
      lds_dma4(a.gidx + lane, idx_dummy);
    }
  };

  f32x16 acc[NB][MB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[nb][mb][v] = 0.0f;
  u32x4 fa[2][MB], fb[2][NB];
  auto frag_one = [&](int slot, auto gc, int i) {  // K-group G of the stage in `slot`
    constexpr int G = decltype(gc)::value;
    const char* st = smem + slot * kW2Stage;
    const int c = 2 * G + (lane >> 5);
    if (i < NB)
      fb[G & 1][i] = *reinterpret_cast<const u32x4*>(st + kW2StageA + wide_off(wn * NB * 32 + i * 32 + (lane & 31), c));
    else
      fa[G & 1][i - NB] = *reinterpret_cast<const u32x4*>(st + wide_off(wm * 64 + (i - NB) * 32 + (lane & 31), c));
  };
  auto mma_one = [&](auto gc, int i) {  // i = nb * MB + mb
    constexpr int G = decltype(gc)::value;
    Mfma<T>::run(fb[G & 1][i / MB], fa[G & 1][i % MB], acc[i / MB][i % MB]);
  };
  using G0 = std::integral_constant<int, 0>;
  using G1 = std::integral_constant<int, 1>;
  using G2 = std::integral_constant<int, 2>;
  using G3 = std::integral_constant<int, 3>;
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;

  // Stage s in slot SL. MODE 0: loads of stage s + 2 in K-group 3; 1: s = S - 2 (no
  // loads); 2: s = S - 1 (no loads, nothing follows). A wave whose rows lack the stage's
  // offset skips its MFMAs and the fragment reads that feed them (they would add zeros);
  // (c_ord, c_kb) is the stage's offset ordinal and K step.
  int c_ord = 0, c_kb = 0;
  auto stage = [&](int SL, auto modec) {
    constexpr int MODE = decltype(modec)::value;
    const int NSL = SL ^ 1;
    const bool on = (pres >> c_ord) & 1u;
    auto group = [&](auto gc, auto mmc, auto frc) {
      constexpr int G = decltype(gc)::value;
      constexpr bool MM = decltype(mmc)::value, FR = decltype(frc)::value;
      wait_lgkm0();
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < NM; ++i) {
        if constexpr (MM) mma_one(gc, i);
        __builtin_amdgcn_sched_barrier(0);
        if (FR && i < NF) {
          if constexpr (G < 3)
            frag_one(SL, std::integral_constant<int, G + 1>{}, i);
          else if constexpr (MODE != 2)
            frag_one(NSL, G0{}, i);
        }
        if constexpr (G == 3 && MODE == 0) issue_load(SL, i);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    using Y = std::true_type;
    using N = std::false_type;
    auto group_on = [&](auto gc) {
      if (on) group(gc, Y{}, Y{});
      else group(gc, N{}, N{});
    };
    group_on(G0{});
    group_on(G1{});
    group_on(G2{});
    if constexpr (MODE != 2) {
      wait_vmcnt<0>();  // stage s + 1 (and the index DMA issued with it) landed
      raw_barrier();
    }
    if constexpr (MODE == 0) cursor_indices();
    // K-group 3 always reads the next stage's first fragments (made conditional on the
    // next stage's offset, the kernel spilled ~570 registers)
    if (on) group(G3{}, Y{}, Y{});
    else group(G3{}, N{}, Y{});
    if constexpr (MODE == 0) advance();
    if (++c_kb == KB) {
      c_kb = 0;
      ++c_ord;
    }
  };

  if (S > 0) {  // S = taps * KB >= 2
    ck = mask ? __builtin_ctz(mask) : 0;
    rest = mask & (mask - 1u);
    ckb = 0;
    cord = 0;
    issue_idx(ck, 0);
    wait_vmcnt<0>();
    raw_barrier();
    // prologue: stages 0 and 1 (the cursor enters offset 0 at stage 0, and offset 1 at
    // stage 1 when KB = 1... KB >= 2 here, so stage 1 is offset 0's second step)
    cursor_indices();
    for (int u = 0; u < L; ++u) issue_load(0, u);
    advance();
    if (S > 1) {
      cursor_indices();
      for (int u = 0; u < L; ++u) issue_load(1, u);
      advance();
    }
    wait_vmcnt<0>();
    raw_barrier();
#pragma unroll
    for (int i = 0; i < NF; ++i) frag_one(0, G0{}, i);

    int slot = 0;
    for (int s = 0; s + 2 < S; ++s) {
      stage(slot, I0{});
      slot ^= 1;
    }
    stage(slot, I1{});
    stage(slot ^ 1, I2{});
  }

  // epilogue: each wave stages its 64 x 128 block
  wait_vmcnt<0>();
  __syncthreads();
  const bool has_bias = a.bias != nullptr;
  constexpr int ROWB = NB * 64, CPR = NB * 4;
  char* stg = smem + wave * (64 * ROWB);
  const int cb = n0 + wn * NB * 32;
  const int64_t out_row_bytes = static_cast<int64_t>(a.cout) * sizeof(T);
  // chunk i of this lane: row lane / CPR + (64 / CPR) i of the wave's rows, 16-byte chunk
  // lane % CPR of its channels; false for rows past the plan or without an output row
  // the output rows of this lane's chunks, all read from LDS at once (one wait, not one
  // per chunk)
  int32_t orow[CPR];
#pragma unroll
  for (int i = 0; i < CPR; ++i) {
    const int tr = wm * 64 + lane / CPR + (64 / CPR) * i;
    const int64_t pt = tile * SUB + tr / kTileRows;
    orow[i] = pt < a.ntiles ? reinterpret_cast<const int32_t*>(rows_lds)[tr] : -1;
  }
  auto chunk_ok = [&](int i) { return orow[i] >= 0 && orow[i] < a.n_out; };
  auto chunk_off = [&](int i) {
    return static_cast<int64_t>(orow[i]) * out_row_bytes + static_cast<int64_t>(cb + (lane % CPR) * 8) * sizeof(T);
  };
  // the residual's chunks are requested before the accumulators are converted and
  // staged, so their latency overlaps that work instead of each group of stores
  u32x4 res[CPR];
  if (a.residual != nullptr) {
#pragma unroll
    for (int i = 0; i < CPR; ++i) res[i] = *reinterpret_cast<const u32x4*>(a.residual + (chunk_ok(i) ? chunk_off(i) : 0));
  }
  // convert (bias, the activation) and stage; the activation is chosen once, outside
  // the element loops
  auto stage_acc = [&](auto silu) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int j0 = nb * 32 + 8 * q + 4 * (lane >> 5);
        float b[4];
        {
          T bt[4];
          __builtin_memcpy(bt, s_bias + ((cb - n0) + j0) * sizeof(T), sizeof(bt));
#pragma unroll
          for (int e = 0; e < 4; ++e) b[e] = has_bias ? to_f32(bt[e]) : 0.0f;
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const int row = mb * 32 + (lane & 31);
          T h[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float x = acc[nb][mb][4 * q + e] + b[e];
            if constexpr (decltype(silu)::value) x = silu_f32(x);
            h[e] = static_cast<T>(x);
          }
          uint2 packed;
          __builtin_memcpy(&packed, h, 8);
          *reinterpret_cast<uint2*>(stg + row * ROWB + (((j0 >> 3) ^ (row & (CPR - 1))) << 4) + (j0 & 4) * 2) = packed;
        }
      }
    }
  };
  if (a.act == HI3D_ACT_SILU) stage_acc(std::true_type{});
  else stage_acc(std::false_type{});
  wait_lgkm0();
  // every staged chunk is read before the first store (one LDS wait)
  u32x4 v[CPR];
#pragma unroll
  for (int i = 0; i < CPR; ++i) {
    const int row = lane / CPR + (64 / CPR) * i;  // 0..63 within this wave's rows
    v[i] = *reinterpret_cast<const u32x4*>(stg + row * ROWB + (((lane % CPR) ^ (row & (CPR - 1))) << 4));
  }
#pragma unroll
  for (int i = 0; i < CPR; ++i) {
    if (a.residual != nullptr) v[i] = add_chunk<T>(v[i], res[i]);
    if (chunk_ok(i)) *reinterpret_cast<u32x4*>(a.out + chunk_off(i)) = v[i];
  }
}

template <typename T>
int launch_wide2(const ConvArgs& base, hipStream_t stream) {
  ConvArgs a = base;
  a.ny = a.cout / 256;
  const int64_t blocks = ceil_div(a.ntiles, 2) * a.ny;
  if (blocks == 0) return HI3D_OK;
  HI3D_REQUIRE(blocks < (int64_t(1) << 31), "too many tiles");
  hipLaunchKernelGGL(conv_wide2_kernel<T>, dim3(static_cast<unsigned>(blocks)), dim3(512), 0, stream, a);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

template <typename T, int BM, int BN, int WGM>
int launch_pipe(const ConvArgs& base, hipStream_t stream) {
  ConvArgs a = base;
  a.ny = static_cast<int32_t>(ceil_div(a.cout, BN));
  const int64_t blocks = ceil_div(a.ntiles, BM / kTileRows) * a.ny;
  if (blocks == 0) return HI3D_OK;
  HI3D_REQUIRE(blocks < (int64_t(1) << 31), "too many tiles");
  hipLaunchKernelGGL((conv_pipe_kernel<T, BM, BN, WGM>), dim3(static_cast<unsigned>(blocks)), dim3(kPipeThreads), 0, stream, a);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

template <typename T>
int launch_mfma(const ConvArgs& base, hipStream_t stream) {
  ConvArgs a = base;
  if constexpr (sizeof(T) == 2) {
    const int rb = a.cin * static_cast<int>(sizeof(T));
    const bool ring_rows = rb % 64 == 0 && rb >= 4 * 64 && rb <= 1024;
    const bool few = a.kvol <= 8 && (rb == 128 || rb == 256) && (a.cout == 64 || a.cout == 128);
    // 8 waves for the large tiles; 128-byte K steps for 128-channel tiles, whose gathers
    // are the larger share of their loads (measured: C128 0.46 vs 0.49 ms, C256 8.8 vs
    // 8.9 ms)
    if (a.kvol <= kMaxPipelinedKvol && rb % 128 == 0 && rb >= 256 && rb <= 1024 && a.cout % 256 == 0)
      return launch_wide2<T>(a, stream);
    if (a.kvol <= kMaxPipelinedKvol && ring_rows && a.cout % 256 == 0) return launch_ring<T, 256, 8>(a, stream);
    // few-offset tables (the strided pair): 128-row tiles in a 48..64 KB ring, so that two
    // or three workgroups share a CU and cover each other's tile start and end
    // 128-byte rows into 128 outputs (the stride-2 down-convolution): one 128-byte
    // request per gathered row, one K stage per offset (0.058-0.062 against 0.064 ms
    // for the 128-row ring tile on one box)
    if (few && rb == 128 && a.cout == 128) return launch_wide<T, 128, 8, true>(a, stream);
    if (few) return a.cout == 64 ? launch_ring<T, 64, 4, 128>(a, stream) : launch_ring<T, 128, 4, 128>(a, stream);
    if (a.kvol <= kMaxPipelinedKvol && ring_rows && a.cout % 128 == 0) {
      if (rb % 128 == 0) return launch_wide<T, 128, 8>(a, stream);
      return launch_ring<T, 128, 8>(a, stream);
    }
    // 64- and 128-channel rows into 64 or 128 outputs: the 128-row ring tiles
    if (a.kvol <= kMaxPipelinedKvol && (rb == 128 || rb == 256) && (a.cout == 64 || a.cout == 128))
      return a.cout == 64 ? launch_ring<T, 64, 4, 128>(a, stream) : launch_ring<T, 128, 4, 128>(a, stream);
  }
  if constexpr (sizeof(T) == 4) {
    // fp32 (four 32x32x2 MFMAs per fragment): 128-row tiles so that small sets still
    // spread over every CU (the 45k-voxel C64 shell makes 353 of them)
    const int rb = a.cin * 4;
    // 64 -> 64 channels: 16-row blocks that skip the offsets absent from their rows;
    // 128-row workgroups over half the output channels (config 1: 0.070 ms; 64-row
    // workgroups over all 64 channels 0.072, 128-row ones 0.082)
    if (a.kvol <= kMaxPipelinedKvol && a.cin == kBlockCin && a.cout == kBlockCout)
      return launch_block_f32<8, 2, 32>(a, stream);
    if (a.kvol <= kMaxPipelinedKvol && rb % 64 == 0 && rb >= 256 && rb <= kRingMaxRowBytes) {
      if (a.cout == 64) return launch_ring<T, 64, 4, 128>(a, stream);
      // 128 x 128 tiles (several column tiles for wider outputs): the largest fp32 tile
      // whose staged output fits the ring (C256: 7.06 -> 6.28 ms, C512: 26.3 -> 24.4 ms
      // against the pipelined kernel on 327,581 voxels)
      if (a.cout % 128 == 0) return launch_ring<T, 128, 4, 128>(a, stream);
    }
  }
  if (a.kvol <= kMaxPipelinedKvol) {
    if (a.cout <= 64) return launch_pipe<T, 256, 64, 8>(a, stream);
    if (a.cout <= 128) return launch_pipe<T, 256, 128, 4>(a, stream);
    return launch_pipe<T, 128, 256, 2>(a, stream);
  }
  int bn;
  const int cout = a.cout;
  if (cout <= 64) bn = 64;
  else if (cout <= 128 || sizeof(T) == 4) bn = 128;
  else bn = 256;
  a.ny = static_cast<int32_t>(ceil_div(cout, bn));
  const int64_t blocks = a.ntiles * a.ny;
  if (blocks == 0) return HI3D_OK;
  HI3D_REQUIRE(blocks < (int64_t(1) << 31), "too many tiles");
  switch (bn) {
    case 64: hipLaunchKernelGGL((conv_mfma_kernel<T, 64>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a); break;
    case 128: hipLaunchKernelGGL((conv_mfma_kernel<T, 128>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a); break;
    default: hipLaunchKernelGGL((conv_mfma_kernel<T, 256>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a); break;
  }
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

template <typename T, typename Acc>
int launch_simple(const void* in, int64_t n_in, int cin, const void* w, const void* bias, int cout, int kvol,
                  const int32_t* table, int64_t n_out, const void* residual, int act, void* out, hipStream_t stream) {
  const int64_t total = n_out * cout;
  if (total == 0) return HI3D_OK;
  hipLaunchKernelGGL((conv_simple_kernel<T, Acc>), dim3(static_cast<unsigned>(ceil_div(total, 256))), dim3(256), 0,
                     stream, static_cast<const T*>(in), n_in, cin, static_cast<const T*>(w),
                     static_cast<const T*>(bias), cout, kvol, table, n_out, static_cast<const T*>(residual), act,
                     static_cast<T*>(out));
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}


// Mean of the present rows of each table row: out[o] = sum_k in[table[o,k]] / (cnt + extra),
// cnt = present entries; fp32 (fp64 for F64) accumulation.
template <typename T, typename Acc>
__global__ void gather_mean_kernel(const T* __restrict__ in, int64_t n_in, int c, const int32_t* __restrict__ table,
                                   int kvol, int64_t n_out, int extra, T* __restrict__ out) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= n_out * c) return;
  const int64_t o = idx / c;
  const int j = static_cast<int>(idx - o * c);
  Acc acc = 0;
  int cnt = 0;
  for (int k = 0; k < kvol; ++k) {
    const int32_t src = table[o * kvol + k];
    if (static_cast<uint64_t>(static_cast<uint32_t>(src)) >= static_cast<uint64_t>(n_in)) continue;
    acc += static_cast<Acc>(in[static_cast<int64_t>(src) * c + j]);
    ++cnt;
  }
  out[idx] = static_cast<T>(acc / static_cast<Acc>(cnt + extra));
}

// The same mean with 16 bytes of a row per thread (rows a multiple of 16 bytes, 16-byte
// aligned): the table entries are read once per chunk instead of once per element, and
// each present row moves in one 16-byte load. Same summation order (present entries in
// table order), so the results equal gather_mean_kernel's.
template <typename T, typename Acc>
__global__ void gather_mean_vec_kernel(const T* __restrict__ in, int64_t n_in, int c, const int32_t* __restrict__ table,
                                       int kvol, int64_t n_out, int extra, T* __restrict__ out) {
  constexpr int E = 16 / static_cast<int>(sizeof(T));
  const int cpr = c / E;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= n_out * cpr) return;
  const int64_t o = idx / cpr;
  const int j = static_cast<int>(idx - o * cpr) * E;
  Acc acc[E];
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0;
  // every entry's load is issued (absent ones read zeros, which leave the sums
  // unchanged: they start at +0 and never become -0), so the loads overlap
  int cnt = 0;
  for (int k0 = 0; k0 < kvol; k0 += 8) {
    uint4 raw[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = k0 + u;
      const int32_t src = k < kvol ? table[o * kvol + k] : -1;
      const bool ok = static_cast<uint64_t>(static_cast<uint32_t>(src)) < static_cast<uint64_t>(n_in);
      cnt += ok ? 1 : 0;
      raw[u] = ok ? *reinterpret_cast<const uint4*>(in + static_cast<int64_t>(src) * c + j) : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const T* v = reinterpret_cast<const T*>(&raw[u]);
#pragma unroll
      for (int e = 0; e < E; ++e) acc[e] += static_cast<Acc>(v[e]);
    }
  }
  uint4 res;
  T* r = reinterpret_cast<T*>(&res);
  const Acc div = static_cast<Acc>(cnt + extra);
#pragma unroll
  for (int e = 0; e < E; ++e) r[e] = static_cast<T>(acc[e] / div);
  *reinterpret_cast<uint4*>(out + o * c + j) = res;
}

template <typename T, typename Acc>
int launch_mean(const void* in, int64_t n_in, int c, const int32_t* table, int kvol, int64_t n_out, int extra, void* out,
                hipStream_t stream) {
  const int64_t total = n_out * c;
  if (total == 0) return HI3D_OK;
  constexpr int E = 16 / static_cast<int>(sizeof(T));
  if (c % E == 0 && ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15) == 0) {
    const int64_t chunks = total / E;
    hipLaunchKernelGGL((gather_mean_vec_kernel<T, Acc>), dim3(static_cast<unsigned>(ceil_div(chunks, 256))), dim3(256),
                       0, stream, static_cast<const T*>(in), n_in, c, table, kvol, n_out, extra, static_cast<T*>(out));
    HI3D_LAUNCH_CHECK();
    return HI3D_OK;
  }
  hipLaunchKernelGGL((gather_mean_kernel<T, Acc>), dim3(static_cast<unsigned>(ceil_div(total, 256))), dim3(256), 0,
                     stream, static_cast<const T*>(in), n_in, c, table, kvol, n_out, extra, static_cast<T*>(out));
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

}  // namespace
}  // namespace hi3d

using namespace hi3d;

extern "C" {

int hi3d_gather_conv(const void* in, int64_t n_in, int32_t cin, const void* weight, const void* bias, int32_t cout,
                     int32_t kvol, const int32_t* rows, const int32_t* gidx, const uint32_t* tile_mask, int64_t n_out,
                     const void* residual, int32_t act, int32_t dtype, void* out, void* stream) {
  const int es = elem_size(dtype);
  HI3D_REQUIRE(es == 2 || es == 4, "gather conv supports F32, F16 and BF16 (got dtype %d)", dtype);
  HI3D_REQUIRE(cin > 0 && cout > 0 && kvol > 0, "channels and kvol must be positive");
  HI3D_REQUIRE((static_cast<int64_t>(cin) * es) % 16 == 0, "cin * element size must be a multiple of 16 bytes");
  HI3D_REQUIRE((static_cast<int64_t>(cout) * es) % 16 == 0, "cout * element size must be a multiple of 16 bytes");
  HI3D_REQUIRE(n_in >= 0 && n_out >= 0, "sizes must be non-negative");
  HI3D_REQUIRE(act == HI3D_ACT_NONE || act == HI3D_ACT_SILU, "unknown activation %d", act);
  if (n_out == 0) return HI3D_OK;
  HI3D_REQUIRE(in && weight && rows && gidx && tile_mask && out, "null pointer argument");
  const uintptr_t align = reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(weight) |
                          reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(residual);
  HI3D_REQUIRE((align & 15) == 0, "feature, weight, residual and output pointers must be 16-byte aligned");
  HI3D_REQUIRE((reinterpret_cast<uintptr_t>(bias) & 3) == 0, "the bias must be 4-byte aligned");
  ConvArgs a{};
  a.in = static_cast<const char*>(in);
  a.n_in = n_in;
  a.cin = cin;
  a.weight = static_cast<const char*>(weight);
  a.bias = bias;
  a.cout = cout;
  a.kvol = kvol;
  a.rows = rows;
  a.gidx = gidx;
  a.tile_mask = tile_mask;
  a.ntiles = ceil_div(n_out, kTileRows);
  a.n_out = n_out;
  a.residual = static_cast<const char*>(residual);
  a.act = act;
  a.out = static_cast<char*>(out);
  hipStream_t s = as_stream(stream);
  switch (dtype) {
    case HI3D_F16: return launch_mfma<_Float16>(a, s);
    case HI3D_BF16: return launch_mfma<__bf16>(a, s);
    default: return launch_mfma<float>(a, s);
  }
}

int hi3d_gather_conv_ln_silu(const void* in, int64_t n_in, int32_t cin, const void* weight, const void* bias,
                             int32_t cout, int32_t kvol, const int32_t* rows, const int32_t* gidx,
                             const uint32_t* tile_mask, int64_t n_out, const int32_t* coords, int32_t batches,
                             const void* scale1p, const void* shift, float eps, void* out, void* stream) {
  const int rb = cin * 2;
  HI3D_REQUIRE(cout == 128, "the fused row norm takes 128 output channels (got %d)", cout);
  HI3D_REQUIRE(rb % 128 == 0 && rb >= 256 && rb <= 1024, "the fused row norm takes 128..512 fp16 input channels in "
               "steps of 64 (got %d)", cin);
  HI3D_REQUIRE(kvol > 0 && kvol <= kMaxPipelinedKvol, "kvol must be 1..%d", kMaxPipelinedKvol);
  HI3D_REQUIRE(n_in >= 0 && n_out >= 0 && batches > 0, "sizes must be non-negative and batches positive");
  if (n_out == 0) return HI3D_OK;
  HI3D_REQUIRE(in && weight && rows && gidx && tile_mask && coords && scale1p && shift && out, "null pointer argument");
  const uintptr_t align = reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(weight) |
                          reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(scale1p) |
                          reinterpret_cast<uintptr_t>(shift);
  HI3D_REQUIRE((align & 15) == 0, "feature, weight, output, scale and shift pointers must be 16-byte aligned");
  HI3D_REQUIRE((reinterpret_cast<uintptr_t>(bias) & 3) == 0, "the bias must be 4-byte aligned");
  ConvArgs a{};
  a.in = static_cast<const char*>(in);
  a.n_in = n_in;
  a.cin = cin;
  a.weight = static_cast<const char*>(weight);
  a.bias = bias;
  a.cout = cout;
  a.kvol = kvol;
  a.rows = rows;
  a.gidx = gidx;
  a.tile_mask = tile_mask;
  a.ntiles = ceil_div(n_out, kTileRows);
  a.n_out = n_out;
  a.act = HI3D_ACT_NONE;
  a.out = static_cast<char*>(out);
  a.ln_coords = coords;
  a.ln_scale = scale1p;
  a.ln_shift = shift;
  a.ln_batches = batches;
  a.ln_eps = eps;
  return launch_wide<_Float16, 128, 8, false, true>(a, as_stream(stream));
}

int hi3d_gather_conv_simple(const void* in, int64_t n_in, int32_t cin, const void* weight, const void* bias,
                            int32_t cout, int32_t kvol, const int32_t* table, int64_t n_out, const void* residual,
                            int32_t act, int32_t dtype, void* out, void* stream) {
  HI3D_REQUIRE(elem_size(dtype) > 0, "unknown dtype %d", dtype);
  HI3D_REQUIRE(cin > 0 && cout > 0 && kvol > 0, "channels and kvol must be positive");
  HI3D_REQUIRE(n_in >= 0 && n_out >= 0, "sizes must be non-negative");
  HI3D_REQUIRE(act == HI3D_ACT_NONE || act == HI3D_ACT_SILU, "unknown activation %d", act);
  if (n_out == 0) return HI3D_OK;
  HI3D_REQUIRE(in && weight && table && out, "null pointer argument");
  hipStream_t s = as_stream(stream);
  switch (dtype) {
    case HI3D_F16: return launch_simple<_Float16, float>(in, n_in, cin, weight, bias, cout, kvol, table, n_out, residual, act, out, s);
    case HI3D_BF16: return launch_simple<__bf16, float>(in, n_in, cin, weight, bias, cout, kvol, table, n_out, residual, act, out, s);
    case HI3D_F32: return launch_simple<float, float>(in, n_in, cin, weight, bias, cout, kvol, table, n_out, residual, act, out, s);
    default: return launch_simple<double, double>(in, n_in, cin, weight, bias, cout, kvol, table, n_out, residual, act, out, s);
  }
}

int hi3d_gather_mean(const void* in, int64_t n_in, int32_t c, const int32_t* table, int32_t kvol, int64_t n_out,
                     int32_t extra, int32_t dtype, void* out, void* stream) {
  HI3D_REQUIRE(elem_size(dtype) > 0, "unknown dtype %d", dtype);
  HI3D_REQUIRE(c > 0 && kvol > 0 && n_in >= 0 && n_out >= 0 && extra >= 0, "bad sizes");
  if (n_out == 0) return HI3D_OK;
  HI3D_REQUIRE(in && table && out, "null pointer argument");
  hipStream_t s = as_stream(stream);
  switch (dtype) {
    case HI3D_F16: return launch_mean<_Float16, float>(in, n_in, c, table, kvol, n_out, extra, out, s);
    case HI3D_BF16: return launch_mean<__bf16, float>(in, n_in, c, table, kvol, n_out, extra, out, s);
    case HI3D_F32: return launch_mean<float, float>(in, n_in, c, table, kvol, n_out, extra, out, s);
    default: return launch_mean<double, double>(in, n_in, c, table, kvol, n_out, extra, out, s);
  }
}

}  // extern "C"
