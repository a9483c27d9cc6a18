// Top-k weighted combine of the grouped expert outputs (plus shared experts).
// 8 columns per thread, fixed summation order (slots ascending, split-K
// slices ascending), no atomics: bit-reproducible.
#include <algorithm>

#include "combine.h"

namespace moeq {

// One 64-thread block per (token, 512-column block); each thread sums 8
// columns of one token (combine_point).
template <int YDT, int SPG>
__global__ __launch_bounds__(64) void combine_kernel(
    const void *y, int splits, int64_t split_stride, int64_t ldy, const int32_t *inv_perm,
    const float *w, int64_t T, int k, int n_shared, int H, int64_t R, void *out, int out_dtype) {
  const int ncb = (H + 511) / 512;
  for (int64_t blk = blockIdx.x; blk < T * ncb; blk += gridDim.x) {
    const int64_t t = blk / ncb;
    const int c = int(blk % ncb) * 512 + 8 * threadIdx.x;
    if (c >= H) continue;
    float acc[8];
    combine_point<YDT, SPG>(y, splits, split_stride, ldy, inv_perm, w, T, k, n_shared, R, t, c, acc);
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
