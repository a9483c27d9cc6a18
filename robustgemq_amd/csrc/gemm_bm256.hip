// Grouped GEMM instantiations for 256-row tiles: one four-wave work-group
// per CU, accumulators in AGPRs (see gemm_wide.h).
#include "gemm_wide.h"

namespace moeq {

template <bool SILU, int ODT>
static int launch_wide(const GemmArgs &g0, int max_tiles, int splits, hipStream_t s) {
  using S = Shape<256, SILU>;
  static_assert(S::NW == 4, "the 256-row tile runs four waves");
  GemmArgs g = g0;
  g.n_ntiles = int(cdiv(g.N, tile_cols<S, false>()));
  const int64_t blocks = int64_t(max_tiles) * g.n_ntiles;
  if (blocks > 0x7fffffff) return fail(MOEQ_ERR_UNSUPPORTED, "grouped_gemm: grid too large");
  dim3 grid(unsigned(blocks), 1, unsigned(splits)), block(S::NW * 64);
  wide_gemm_kernel<S::NB, SILU ? 2 : 1, SILU ? MOEQ_EPI_SILU_MUL : MOEQ_EPI_STORE, ODT, 16, 1><<<grid, block, 0, s>>>(g);
  return check_launch("grouped_gemm");
}

template <>
int launch_grouped_gemm<256>(const GemmArgs &g, bool silu, int a_dtype, int out_dtype, int max_tiles,
                            int splits, hipStream_t s) {
  // rows are copied global -> LDS as they are, so activations must be F16
  if (a_dtype != MOEQ_F16) return fail(MOEQ_ERR_UNSUPPORTED, "grouped_gemm: bm=256 needs F16 activations");
  if (silu) return launch_wide<true, MOEQ_F16>(g, max_tiles, splits, s);
  if (out_dtype == MOEQ_F32) return launch_wide<false, MOEQ_F32>(g, max_tiles, splits, s);
  return launch_wide<false, MOEQ_F16>(g, max_tiles, splits, s);
}

}  // namespace moeq
