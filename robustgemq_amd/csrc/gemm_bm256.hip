// Grouped GEMM instantiations for 256-row tiles (see gemm_impl.h).
#include "gemm_impl.h"

namespace moeq {

template <>
int launch_grouped_gemm<256>(const GemmArgs &g, bool silu, int a_dtype, int out_dtype, int max_tiles,
                            int splits, hipStream_t s) {
  // rows are copied global -> LDS as they are, so activations must be F16
  if (a_dtype != MOEQ_F16) return fail(MOEQ_ERR_UNSUPPORTED, "grouped_gemm: bm=256 needs F16 activations");
  if (silu) return launch_one<256, true, MOEQ_F16, MOEQ_F16>(g, max_tiles, splits, s);
  if (out_dtype == MOEQ_F32) return launch_one<256, false, MOEQ_F16, MOEQ_F32>(g, max_tiles, splits, s);
  return launch_one<256, false, MOEQ_F16, MOEQ_F16>(g, max_tiles, splits, s);
}

}  // namespace moeq
