// Shared definitions for the gfx950 kernels of libmoeq.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moeq.h"

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

namespace moeq {

// ---------------------------------------------------------------- errors
// Records a message for moeq_last_error() and returns `code`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Returns MOEQ_OK, or MOEQ_ERR_HIP with the message of the pending launch error.
int check_launch(const char *what);

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// Row capacity of one grouped-GEMM tile of class bm: the schedule splits an
// expert's m rows into ceil(m / cap) tiles, so the prefill classes leave room
// above their nominal height (an expert a little past 2 x 128 rows still
// takes two tiles, not three).  0 for an unknown class.
__host__ __device__ constexpr int tile_rows(int bm) {
  return bm == 16 ? 32 : bm == 32 ? 48 : bm == 64 ? 96 : bm == 128 ? 160 : bm == 256 ? 256 : 0;
}

// The grouped GEMM instantiates, per class, kernel variants for 16-row block
// counts {1, 2} (bm 16), {2, 3} (32), {2, 4, 6} (64), {2, 4, 8, 10} (128) and
// {2, 4, 8, 10, 16} (256); a tile of b blocks runs the smallest count >= b.
// The schedule cuts experts into tiles of the largest count and of the one
// below it, returned here (for bm 256, 10: an expert of 17..20 blocks takes two
// tiles of about half, not 16 blocks and a remainder).
__host__ __device__ constexpr int tile_blocks_below(int bm) {
  return bm == 16 ? 1 : bm == 32 ? 2 : bm == 64 ? 4 : bm == 128 ? 8 : bm == 256 ? 10 : 0;
}

// The variant below tile_blocks_below(bm) (0 where that is the smallest):
// the schedule lists tiles of more blocks than tile_blocks_below first, then
// those of more than this, then the rest.
__host__ __device__ constexpr int tile_blocks_below2(int bm) {
  return bm == 64 ? 2 : bm == 128 ? 4 : bm == 256 ? 8 : 0;
}

// ------------------------------------------------------- device helpers
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(uint32_t(b) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  f16 h = (f16)f;  // v_cvt_f16_f32, round to nearest even
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  return (float)__builtin_bit_cast(f16, b);
}

// Loads element i of a row stored as f16 / bf16 / f32 and widens it exactly.
__device__ __forceinline__ float load_as_f32(const void *p, int dtype, int64_t i) {
  if (dtype == MOEQ_F32) return static_cast<const float *>(p)[i];
  uint16_t b = static_cast<const uint16_t *>(p)[i];
  return dtype == MOEQ_BF16 ? bf16_to_f32(b) : f16_bits_to_f32(b);
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// silu(g) * u in fp32: the gate/up epilogue and moeq_silu_mul share it.
__device__ __forceinline__ float silu_mul(float g, float u) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

}  // namespace moeq
