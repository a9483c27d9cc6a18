// Grouped GEMM dispatch for 16-row tiles; the launches are instantiated in
// gemm_bm16_silu.hip, gemm_bm16_f16.hip and gemm_bm16_f32.hip.
#include "gemm_impl.h"

namespace moeq {

template <int ADT, int ODT, bool SILU>
int launch16(const GemmArgs &g, int max_tiles, int splits, hipStream_t s);

template <>
int launch_grouped_gemm<16>(const GemmArgs &g, bool silu, int a_dtype, int out_dtype, int max_tiles,
                            int splits, hipStream_t s) {
  const bool bf = a_dtype == MOEQ_BF16;
  if (silu) return bf ? launch16<MOEQ_BF16, MOEQ_F16, true>(g, max_tiles, splits, s)
                      : launch16<MOEQ_F16, MOEQ_F16, true>(g, max_tiles, splits, s);
  if (out_dtype == MOEQ_F32)
    return bf ? launch16<MOEQ_BF16, MOEQ_F32, false>(g, max_tiles, splits, s)
              : launch16<MOEQ_F16, MOEQ_F32, false>(g, max_tiles, splits, s);
  return bf ? launch16<MOEQ_BF16, MOEQ_F16, false>(g, max_tiles, splits, s)
            : launch16<MOEQ_F16, MOEQ_F16, false>(g, max_tiles, splits, s);
}

}  // namespace moeq
