// Combine arithmetic shared by combine_kernel and the decode down
// projection's fused tail (gemm_impl.h): one output point, token t and
// columns c .. c + 7, summed in a fixed order (slots ascending, split-K
// slices ascending, shared experts last) with no atomics, so both paths give
// the same bits.
#pragma once

#include "common.h"

namespace moeq {

constexpr int kCombineSlots = 16;  // top_k covered by the batched-load path

template <int YDT>
__device__ __forceinline__ void load_y8(const void *y, int64_t off, float (&v)[8]) {
  if constexpr (YDT == MOEQ_F32) {
    const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(y) + off);
    float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    uint4 u = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(y) + off);
    uint32_t ws[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = f16_bits_to_f32(uint16_t(ws[j] & 0xffffu));
      v[2 * j + 1] = f16_bits_to_f32(uint16_t(ws[j] >> 16));
    }
  }
}

// Output store of 8 columns.
__device__ __forceinline__ void store8(void *out, int out_dtype, int64_t o, const float (&acc)[8]) {
  if (out_dtype == MOEQ_F32) {
    float4 *p = reinterpret_cast<float4 *>(static_cast<float *>(out) + o);
    p[0] = (float4){acc[0], acc[1], acc[2], acc[3]};
    p[1] = (float4){acc[4], acc[5], acc[6], acc[7]};
  } else {
    uint32_t ws[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint16_t lo, hi;
      if (out_dtype == MOEQ_BF16) {
        lo = f32_to_bf16(acc[2 * j]);
        hi = f32_to_bf16(acc[2 * j + 1]);
      } else {
        lo = f32_to_f16_bits(acc[2 * j]);
        hi = f32_to_f16_bits(acc[2 * j + 1]);
      }
      ws[j] = uint32_t(lo) | (uint32_t(hi) << 16);
    }
    *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(out) + o) = (uint4){ws[0], ws[1], ws[2], ws[3]};
  }
}


// acc = fma(w_s, (0 + y_s,0 + y_s,1 + ...), acc) over the token's slots
// s = 0 .. k-1, then + the shared experts' rows.  SPG > 0 (splits == SPG,
// k <= kCombineSlots): the rows and weights of all slots are read in one
// round trip, then the y slices of 8 / SPG slots at a time are all in flight
// before the first is summed (slots past k, and invalid rows, read row 0 and
// are not added).  SPG == 0: any split count, one slot at a time.
template <int YDT, int SPG>
__device__ __forceinline__ void combine_point(const void *y, int splits, int64_t split_stride, int64_t ldy,
                                              const int32_t *inv_perm, const float *w, int64_t T, int k,
                                              int n_shared, int64_t R, int64_t t, int c, float (&acc)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.f;
  if constexpr (SPG > 0) {
    constexpr int G = 8 / SPG;
    int rr[kCombineSlots];
    float ww[kCombineSlots];
#pragma unroll
    for (int s = 0; s < kCombineSlots; ++s) {
      const int sc = min(s, k - 1);
      rr[s] = inv_perm[t * k + sc];
      ww[s] = w[t * k + sc];
    }
#pragma unroll
    for (int s0 = 0; s0 < kCombineSlots; s0 += G) {
      if (s0 >= k) break;
      float v[G][SPG][8];
      bool ok[G];
#pragma unroll
      for (int u = 0; u < G; ++u) {
        ok[u] = s0 + u < k && rr[s0 + u] >= 0 && rr[s0 + u] < R;
        const int64_t r = ok[u] ? rr[s0 + u] : 0;
#pragma unroll
        for (int sp = 0; sp < SPG; ++sp) load_y8<YDT>(y, sp * split_stride + r * ldy + c, v[u][sp]);
      }
#pragma unroll
      for (int u = 0; u < G; ++u) {
        if (!ok[u]) continue;
        float sum[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int sp = 0; sp < SPG; ++sp)
#pragma unroll
          for (int j = 0; j < 8; ++j) sum[j] += v[u][sp][j];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = __builtin_fmaf(ww[s0 + u], sum[j], acc[j]);
      }
    }
  } else {
    for (int s = 0; s < k; ++s) {
      const int32_t r = inv_perm[t * k + s];
      if (r < 0 || r >= R) continue;  // never for a schedule from moeq_permute
      const float wt = w[t * k + s];
      float sum[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int sp = 0; sp < splits; ++sp) {
        float v[8];
        load_y8<YDT>(y, sp * split_stride + int64_t(r) * ldy + c, v);
#pragma unroll
        for (int j = 0; j < 8; ++j) sum[j] += v[j];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = __builtin_fmaf(wt, sum[j], acc[j]);
    }
  }
  for (int v = 0; v < n_shared; ++v) {
    const int64_t r = T * k + int64_t(v) * T + t;
    for (int sp = 0; sp < splits; ++sp) {
      float y8[8];
      load_y8<YDT>(y, sp * split_stride + r * ldy + c, y8);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += y8[j];
    }
  }
}

}  // namespace moeq
