// Tile constants and MFMA fragment helpers shared by the gather convolution and the
// int8 GEMM. All matrix tiles in LDS use one layout: a row of 128 bytes (one K-block)
// split into eight 16-byte chunks, chunk c of row r stored at position
// c ^ ((r >> 1) & 7). For a fixed logical chunk, any 16 consecutive rows then fall in
// 16 distinct 4-bank groups, so the ds_read_b128 fragment reads of the 32x32 MFMAs and
// the row-wise ds_write_b128 stores are free of bank conflicts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace hi3d {

constexpr int kTileRows = 128;  // output rows per convolution tile

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// The residual add of the convolution epilogues on a 16-byte chunk: T(float(v) +
// float(r)) per element. fp16 chunks add as 8 native fp16 adds (4 packed ops against 4
// ops per element): fp32's 24 bits are at least 2 * 11 + 2, so the sum of two fp16
// values rounded through fp32 and rounded once to fp16 agree.
template <typename T>
__device__ __forceinline__ u32x4 add_chunk(u32x4 v, u32x4 r) {
  if constexpr (std::is_same_v<T, _Float16>) {
#pragma clang fp contract(off)
    return __builtin_bit_cast(u32x4, __builtin_bit_cast(f16x8, v) + __builtin_bit_cast(f16x8, r));
  } else {
    constexpr int kElems = 16 / static_cast<int>(sizeof(T));
    T* pv = reinterpret_cast<T*>(&v);
    const T* pr = reinterpret_cast<const T*>(&r);
#pragma unroll
    for (int e = 0; e < kElems; ++e) pv[e] = static_cast<T>(static_cast<float>(pv[e]) + static_cast<float>(pr[e]));
    return v;
  }
}

// SiLU of the convolution epilogues in fp32: x * sigmoid(x) with the sigmoid through the
// hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32; ~1 ulp each), 4 vector ops against
// ~25 for expf and a correctly rounded division. Within a few fp32 ulps of
// x / (1 + e^-x); where the output is then rounded to 16 bits, that moves the last bit
// of about one output in 10^4.
__device__ __forceinline__ float silu_f32(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

__device__ __forceinline__ int lds_offset(int row, int chunk) {
  return row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4);
}

// One 32-byte K-group of a 32x32 output block: lane l supplies 16 bytes of row
// (l % 32) from logical chunk (2g + l / 32) for both operands.
template <typename T>
struct Mfma;

template <>
struct Mfma<_Float16> {
  __device__ __forceinline__ static void run(u32x4 a, u32x4 b, f32x16& c) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

template <>
struct Mfma<__bf16> {
  __device__ __forceinline__ static void run(u32x4 a, u32x4 b, f32x16& c) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                0);
  }
};

// fp32: the 16-byte fragment holds 4 consecutive K values; four 32x32x2 MFMAs consume
// them (both operands use the same K permutation, so the contraction is unchanged).
// The whole vector is bit-cast before indexing: bit-casting a single component
// (`__builtin_bit_cast(float, a.y)`) is compiled as a read of component 0 by this
// toolchain.
template <>
struct Mfma<float> {
  __device__ __forceinline__ static void run(u32x4 a, u32x4 b, f32x16& c) {
    const f32x4 af = __builtin_bit_cast(f32x4, a), bf = __builtin_bit_cast(f32x4, b);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(af[0], bf[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(af[1], bf[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(af[2], bf[2], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(af[3], bf[3], c, 0, 0, 0);
  }
};

// Row of accumulator element v of a 32x32 block held by `lane` (column = lane % 32).
__device__ __forceinline__ int acc_row(int lane, int v) { return ((v >> 2) << 3) + ((lane >> 5) << 2) + (v & 3); }

// s_waitcnt with only the vector-memory counter limited to N outstanding operations
// (fields: vmcnt[3:0], expcnt[6:4] = 7, lgkmcnt[11:8] = 15, vmcnt[5:4] at bits 15:14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Wait for this wave's LDS operations only (vmcnt left at its maximum, 63).
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14)); }

// Workgroup barrier without the implicit drain of outstanding global loads that
// __syncthreads() performs; the empty asm statements keep the compiler from moving
// memory accesses across it. Callers wait for their own operations first.
__device__ __forceinline__ void raw_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// 16-byte direct-to-LDS load (global_load_lds_dwordx4): lane l's 16 bytes land at
// lds_wave_base + 16 l. The LDS base must be the same for the whole wave.
__device__ __forceinline__ void lds_dma16(const void* src, char* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(lds_wave_base), 16, 0, 0);
}

// 4-byte direct-to-LDS load (global_load_lds_dword): lane l's 4 bytes land at
// lds_wave_base + 4 l.
__device__ __forceinline__ void lds_dma4(const void* src, char* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(lds_wave_base), 4, 0, 0);
}

// XCD-aware block order: the chip deals workgroups round-robin over its 8 XCDs, so
// block b runs on XCD b % 8. Remap so each XCD walks a contiguous range of work items
// (neighbouring tiles share gathered rows and weights in that XCD's L2).
__device__ __forceinline__ int64_t xcd_remap(int64_t b, int64_t total) {
  const int64_t per = total / 8, rem = total % 8;
  const int64_t xcd = b % 8, local = b / 8;
  return xcd * per + (xcd < rem ? xcd : rem) + local;
}

}  // namespace hi3d
