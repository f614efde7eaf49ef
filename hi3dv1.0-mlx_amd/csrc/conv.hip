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
#include "common.h"
#include "conv_tile.h"

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
  int32_t ny;  // column tiles
  const char* residual;
  int32_t act;
  char* out;
};

template <typename T>
__device__ __forceinline__ float to_f32(T v) {
  return static_cast<float>(v);
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

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
        if (a.act == HI3D_ACT_SILU) x = silu(x);
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
    if (orow < 0 || ncol >= a.cout) continue;
    u32x4 v = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(C) + (i * BN + cc * EPC) * sizeof(T));
    const int64_t off = static_cast<int64_t>(orow) * out_row_bytes + static_cast<int64_t>(ncol) * sizeof(T);
    if (a.residual != nullptr) {
      u32x4 r = *reinterpret_cast<const u32x4*>(a.residual + off);
      T* pv = reinterpret_cast<T*>(&v);
      const T* pr = reinterpret_cast<const T*>(&r);
#pragma unroll
      for (int e = 0; e < EPC; ++e) pv[e] = static_cast<T>(to_f32(pv[e]) + to_f32(pr[e]));
    }
    *reinterpret_cast<u32x4*>(a.out + off) = v;
  }
}

// ------------------------------------------------------------------------------------
// Pipelined variant for kernel volumes up to 27 (3^3 submanifold, 2^3 strided pair).
//
// Stages are (present offset, 128-byte K-block) pairs, so every gathered row moves as
// whole 128-byte lines. Both operands travel global -> LDS by direct-to-LDS 16-byte loads
// (global_load_lds_dwordx4, no register staging): gathered rows (A) run two stages
// ahead in a 3-deep ring, weights (B, L2-resident) one stage ahead in a 2-deep ring.
// Each iteration issues B(s+1) then A(s+2), so waiting until only the newest A group
// is outstanding completes both A(s) and B(s); the barrier after the wait publishes
// every wave's part. Absent rows and K padding load from a zero buffer. The tile's
// gather indices (all offsets, [K][BM]) are copied to LDS once per tile and read into
// registers once per offset. Fragment reads run two K-groups ahead of the MFMAs.
// A BM-row tile covers BM / 128 consecutive plan tiles (union of their masks).

__device__ __attribute__((aligned(16))) const uint32_t g_zero16[4] = {0u, 0u, 0u, 0u};

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
  // s_waitcnt: vmcnt[3:0] | expcnt[6:4] (7 = no wait) | lgkmcnt[11:8] (15 = no wait) | vmcnt[5:4] at [15:14]
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ void lds_dma16(const void* src, char* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(lds_wave_base), 16, 0, 0);
}

constexpr int kMaxPipelinedKvol = 27;

template <typename T, int BM, int BN, int WGM>
__global__ __launch_bounds__(256) void conv_pipe_kernel(ConvArgs a) {
  constexpr int WGN = 4 / WGM;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int MB = WM / 32, NB = WN / 32;
  constexpr int A_INS = BM / 32, B_INS = BN / 32;  // 16-byte loads per thread per stage
  constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128;
  constexpr int PIPE = 3 * A_BYTES + 2 * B_BYTES;
  constexpr int EPI = BM * BN * static_cast<int>(sizeof(T));
  constexpr int REGION = PIPE > EPI ? PIPE : EPI;
  constexpr int SUB = BM / kTileRows;
  static_assert(A_INS >= 1 && B_INS >= 1 && MB >= 1 && NB >= 1, "tile shape");
  __shared__ __attribute__((aligned(16))) char smem[REGION + BM * kMaxPipelinedKvol * 4];
  char* const ring_a = smem;
  char* const ring_b = smem + 3 * A_BYTES;
  int32_t* const gidx = reinterpret_cast<int32_t*>(smem + REGION);

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

  // gather indices of the tile, all offsets: LDS [k][BM]
  {
    const int per_k = BM / 4;
    for (int q = tid; q < kvol * per_k; q += 256) {
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
  const int lrow = lane >> 3;  // row of this lane within an 8-row load group

  struct Iter {
    int k, kb;
    uint32_t rest;
  };
  auto first = [&]() {
    Iter it;
    it.k = mask ? __builtin_ctz(mask) : 0;
    it.kb = 0;
    it.rest = mask & (mask - 1u);
    return it;
  };
  auto advance = [&](Iter& it) {
    if (++it.kb == nkb) {
      it.kb = 0;
      it.k = it.rest ? __builtin_ctz(it.rest) : it.k;
      it.rest &= it.rest - 1u;
    }
  };
  Iter ia = first(), ib = first();
  int sa = 0, sb = 0;  // next stage to issue for A / B

  // gather rows of the current A tap, read from LDS once per tap (all K-blocks reuse them)
  int32_t asrc[A_INS];
  auto load_asrc = [&]() {
    const int32_t* g = gidx + ia.k * BM;
#pragma unroll
    for (int j = 0; j < A_INS; ++j) asrc[j] = g[(j * 4 + wave) * 8 + lrow];
  };
  auto issue_a = [&]() {
    char* A = ring_a + (sa % 3) * A_BYTES;
    if (ia.kb == 0) load_asrc();
#pragma unroll
    for (int j = 0; j < A_INS; ++j) {
      const int grp = j * 4 + wave;
      const int row = grp * 8 + lrow;
      const int c = (lane & 7) ^ ((row >> 1) & 7);  // logical chunk landing at this lane's slot
      const int cidx = ia.kb * 8 + c;
      const int32_t src = asrc[j];
      const bool ok = cidx < row_chunks && static_cast<uint64_t>(static_cast<uint32_t>(src)) < n_in;
      const char* real = a.in + static_cast<int64_t>(ok ? src : 0) * row_bytes + cidx * 16;
      lds_dma16(ok ? static_cast<const void*>(real) : static_cast<const void*>(g_zero16), A + grp * 1024);
    }
    advance(ia);
    ++sa;
  };
  auto issue_b = [&]() {
    char* B = ring_b + (sb % 2) * B_BYTES;
#pragma unroll
    for (int j = 0; j < B_INS; ++j) {
      const int grp = j * 4 + wave;
      const int row = grp * 8 + lrow;
      const int c = (lane & 7) ^ ((row >> 1) & 7);
      const int cidx = ib.kb * 8 + c;
      const int n = n0 + row;
      const bool ok = cidx < row_chunks && n < a.cout;
      const char* real = a.weight + (static_cast<int64_t>(ok ? n : 0) * kvol + ib.k) * row_bytes + cidx * 16;
      lds_dma16(ok ? static_cast<const void*>(real) : static_cast<const void*>(g_zero16), B + grp * 1024);
    }
    advance(ib);
    ++sb;
  };

  f32x16 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mb][nb][v] = 0.0f;

  auto compute = [&](int s) {
    const char* A = ring_a + (s % 3) * A_BYTES;
    const char* B = ring_b + (s % 2) * B_BYTES;
    // fragment reads run two K-groups ahead of the MFMAs (at most 12 reads in flight,
    // within the 4-bit LDS counter), so each K-group waits only for its own reads
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
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) Mfma<T>::run(af[g][mb], bf[g][nb], acc[mb][nb]);
    };
    frags(0);
    frags(1);
    __builtin_amdgcn_sched_barrier(0);
    mma(0);
    __builtin_amdgcn_sched_barrier(0);
    frags(2);
    __builtin_amdgcn_sched_barrier(0);
    mma(1);
    __builtin_amdgcn_sched_barrier(0);
    frags(3);
    __builtin_amdgcn_sched_barrier(0);
    mma(2);
    __builtin_amdgcn_sched_barrier(0);
    mma(3);
  };

  if (S > 0) {
    issue_b();
    issue_a();
    if (S > 1) issue_a();
  }
  for (int s = 0; s < S; ++s) {
    if (s + 1 < S) wait_vmcnt<A_INS>();
    else wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    if (s + 1 < S) issue_b();
    if (s + 2 < S) issue_a();
    compute(s);
  }
  __syncthreads();

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
        const int i = wm * WM + mb * 32 + acc_row(lane, v);
        float x = acc[mb][nb][v] + b;
        if (a.act == HI3D_ACT_SILU) x = silu(x);
        C[i * BN + j] = static_cast<T>(x);
      }
    }
  }
  __syncthreads();
  constexpr int EPC = 16 / static_cast<int>(sizeof(T));
  constexpr int CPR = BN / EPC;
  const int64_t out_row_bytes = static_cast<int64_t>(a.cout) * sizeof(T);
  for (int q = tid; q < BM * CPR; q += 256) {
    const int i = q / CPR, cc = q - (q / CPR) * CPR;
    const int64_t pt = tile * SUB + i / kTileRows;
    if (pt >= a.ntiles) continue;
    const int32_t orow = a.rows[pt * kTileRows + (i % kTileRows)];
    const int ncol = n0 + cc * EPC;
    if (orow < 0 || ncol >= a.cout) continue;
    u32x4 v = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(C) + (i * BN + cc * EPC) * sizeof(T));
    const int64_t off = static_cast<int64_t>(orow) * out_row_bytes + static_cast<int64_t>(ncol) * sizeof(T);
    if (a.residual != nullptr) {
      u32x4 r = *reinterpret_cast<const u32x4*>(a.residual + off);
      T* pv = reinterpret_cast<T*>(&v);
      const T* pr = reinterpret_cast<const T*>(&r);
#pragma unroll
      for (int e = 0; e < EPC; ++e) pv[e] = static_cast<T>(to_f32(pv[e]) + to_f32(pr[e]));
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

template <typename T, int BM, int BN, int WGM>
int launch_dma(const ConvArgs& base, hipStream_t stream) {
  ConvArgs a = base;
  a.ny = static_cast<int32_t>(ceil_div(a.cout, BN));
  const int64_t blocks = ceil_div(a.ntiles, BM / kTileRows) * a.ny;
  if (blocks == 0) return HI3D_OK;
  HI3D_REQUIRE(blocks < (int64_t(1) << 31), "too many tiles");
  hipLaunchKernelGGL((conv_pipe_kernel<T, BM, BN, WGM>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a);
  HI3D_LAUNCH_CHECK();
  return HI3D_OK;
}

template <typename T>
int launch_mfma(const ConvArgs& base, hipStream_t stream) {
  ConvArgs a = base;
  if (a.kvol <= kMaxPipelinedKvol) {
    if (a.cout <= 64) return launch_dma<T, 256, 64, 4>(a, stream);
    if (sizeof(T) == 4) return launch_dma<T, 128, 128, 2>(a, stream);
    if (a.cout <= 128) return launch_dma<T, 256, 128, 4>(a, stream);
    return launch_dma<T, 128, 256, 2>(a, stream);
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

template <typename T, typename Acc>
int launch_mean(const void* in, int64_t n_in, int c, const int32_t* table, int kvol, int64_t n_out, int extra, void* out,
                hipStream_t stream) {
  const int64_t total = n_out * c;
  if (total == 0) return HI3D_OK;
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
