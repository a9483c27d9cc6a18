// Grouped GEMM instantiations for 16-row tiles (see gemm_impl.h).
#include "gemm_impl.h"

namespace moeq {

template <>
int launch_grouped_gemm<16>(const GemmArgs &g, bool silu, int a_dtype, int out_dtype, int max_tiles,
                            int splits, hipStream_t s) {
  const bool bf = a_dtype == MOEQ_BF16;
  if (silu) return bf ? launch_one<16, true, MOEQ_BF16, MOEQ_F16>(g, max_tiles, splits, s)
                      : launch_one<16, true, MOEQ_F16, MOEQ_F16>(g, max_tiles, splits, s);
  if (out_dtype == MOEQ_F32)
    return bf ? launch_one<16, false, MOEQ_BF16, MOEQ_F32>(g, max_tiles, splits, s)
              : launch_one<16, false, MOEQ_F16, MOEQ_F32>(g, max_tiles, splits, s);
  return bf ? launch_one<16, false, MOEQ_BF16, MOEQ_F16>(g, max_tiles, splits, s)
            : launch_one<16, false, MOEQ_F16, MOEQ_F16>(g, max_tiles, splits, s);
}

}  // namespace moeq
