// Top-k weighted combine of the grouped expert outputs (plus shared experts).
// 8 columns per thread, fixed summation order (slots ascending, split-K
// slices ascending), no atomics: bit-reproducible.
#include <algorithm>

#include "common.h"

namespace moeq {

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

constexpr int kCombineSlots = 16;  // top_k covered by the batched-load kernel

// One 64-thread block per (token, 512-column block); each thread sums 8
// columns over the token's slots in slot order (split-K slices in order):
//   acc = fma(w_s, (0 + y_s,0 + y_s,1 + ...), acc),  s = 0 .. k-1,
// then adds the shared experts' rows.  SPG > 0 (splits == SPG, top_k <=
// kCombineSlots): the rows and weights of all slots are read in one round
// trip, then the y slices of 8 / SPG slots at a time are all in flight
// before the first is summed (slots past top_k, and invalid rows, read row
// 0 and are not added).  SPG == 0: any split count, one slot at a time.
template <int YDT, int SPG>
__global__ __launch_bounds__(64) void combine_kernel(
    const void *y, int splits, int64_t split_stride, int64_t ldy, const int32_t *inv_perm,
    const float *w, int64_t T, int k, int n_shared, int H, int64_t R, void *out, int out_dtype) {
  const int ncb = (H + 511) / 512;
  for (int64_t blk = blockIdx.x; blk < T * ncb; blk += gridDim.x) {
    const int64_t t = blk / ncb;
    const int c = int(blk % ncb) * 512 + 8 * threadIdx.x;
    if (c >= H) continue;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
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
    store8(out, out_dtype, t * H + c, acc);
  }
}

template <int YDT>
static void launch_combine(dim3 grid, hipStream_t s, const void *y, int splits, int64_t split_stride,
                           int64_t ldy, const int32_t *inv_perm, const float *w, int64_t T, int k,
                           int n_shared, int H, int64_t R, void *out, int out_dtype) {
#define MOEQ_CB(G) \
  combine_kernel<YDT, G><<<grid, dim3(64), 0, s>>>(y, splits, split_stride, ldy, inv_perm, w, T, k, n_shared, H, R, out, out_dtype)
  if (k > kCombineSlots) MOEQ_CB(0);
  else if (splits == 1) MOEQ_CB(1);
  else if (splits == 2) MOEQ_CB(2);
  else if (splits == 4) MOEQ_CB(4);
  else MOEQ_CB(0);
#undef MOEQ_CB
}

}  // namespace moeq

using namespace moeq;

extern "C" int moeq_combine(const void *y, int y_dtype, int splits, int64_t split_stride,
                            int64_t ldy, const int32_t *inv_perm, const float *w, int64_t T,
                            int top_k, int n_shared, int H, void *out, int out_dtype,
                            void *stream) {
  if (!y || !inv_perm || !w || !out) return fail(MOEQ_ERR_INVALID, "combine: null pointer");
  if (y_dtype != MOEQ_F16 && y_dtype != MOEQ_F32) return fail(MOEQ_ERR_INVALID, "combine: y_dtype=%d", y_dtype);
  if (out_dtype != MOEQ_F16 && out_dtype != MOEQ_BF16 && out_dtype != MOEQ_F32)
    return fail(MOEQ_ERR_INVALID, "combine: out_dtype=%d", out_dtype);
  if (T <= 0 || top_k <= 0 || n_shared < 0 || splits < 1)
    return fail(MOEQ_ERR_INVALID, "combine: T=%lld top_k=%d n_shared=%d splits=%d", (long long)T, top_k, n_shared, splits);
  if (H <= 0 || H % 8 || ldy < H || ldy % 8)
    return fail(MOEQ_ERR_INVALID, "combine: H=%d ldy=%lld (multiples of 8, ldy >= H)", H, (long long)ldy);
  if (splits > 1 && split_stride < (T * top_k + int64_t(n_shared) * T) * ldy)
    return fail(MOEQ_ERR_INVALID, "combine: split_stride=%lld too small", (long long)split_stride);
  const int64_t R = T * top_k + int64_t(n_shared) * T;
  const int64_t blocks = T * ((H + 511) / 512);
  dim3 grid(unsigned(std::min<int64_t>(blocks, 1 << 20)));
  hipStream_t s = as_stream(stream);
  if (y_dtype == MOEQ_F32)
    launch_combine<MOEQ_F32>(grid, s, y, splits, split_stride, ldy, inv_perm, w, T, top_k, n_shared, H, R, out,
                             out_dtype);
  else
    launch_combine<MOEQ_F16>(grid, s, y, splits, split_stride, ldy, inv_perm, w, T, top_k, n_shared, H, R, out,
                             out_dtype);
  return check_launch("combine");
}

// ------------------------------------------------------------- SiLU * mul
// out = fp16(silu(x1) * x3), 8 elements per thread, fp32 arithmetic shared
// with the gate/up epilogue (silu_mul in common.h).
__global__ void silu_mul_kernel(const uint16_t *x1, const uint16_t *x3, int64_t n, uint16_t *out) {
  const int64_t i = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 8;
  if (i >= n) return;  // n is a multiple of 8
  const uint4 a = *reinterpret_cast<const uint4 *>(x1 + i);
  const uint4 b = *reinterpret_cast<const uint4 *>(x3 + i);
  const uint32_t wa[4] = {a.x, a.y, a.z, a.w}, wb[4] = {b.x, b.y, b.z, b.w};
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float lo = silu_mul(f16_bits_to_f32(uint16_t(wa[j] & 0xffffu)), f16_bits_to_f32(uint16_t(wb[j] & 0xffffu)));
    const float hi = silu_mul(f16_bits_to_f32(uint16_t(wa[j] >> 16)), f16_bits_to_f32(uint16_t(wb[j] >> 16)));
    o[j] = uint32_t(f32_to_f16_bits(lo)) | (uint32_t(f32_to_f16_bits(hi)) << 16);
  }
  *reinterpret_cast<uint4 *>(out + i) = (uint4){o[0], o[1], o[2], o[3]};
}

extern "C" int moeq_silu_mul(const uint16_t *x1, const uint16_t *x3, int64_t n, uint16_t *out, void *stream) {
  if (!x1 || !x3 || !out) return fail(MOEQ_ERR_INVALID, "silu_mul: null pointer");
  if (n <= 0 || n % 8) return fail(MOEQ_ERR_INVALID, "silu_mul: n=%lld must be a positive multiple of 8", (long long)n);
  const int64_t blocks = cdiv(n / 8, 256);
  if (blocks > 0x7fffffff) return fail(MOEQ_ERR_UNSUPPORTED, "silu_mul: n=%lld too large", (long long)n);
  silu_mul_kernel<<<dim3(unsigned(blocks)), dim3(256), 0, as_stream(stream)>>>(x1, x3, n, out);
  return check_launch("silu_mul");
}
