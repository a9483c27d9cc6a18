// 16-row grouped GEMM launches, fp16-output kernels.
#include "gemm_bm16_impl.h"

namespace moeq {

template int launch16<MOEQ_F16, MOEQ_F16, false>(const GemmArgs &, int, int, hipStream_t);
template int launch16<MOEQ_BF16, MOEQ_F16, false>(const GemmArgs &, int, int, hipStream_t);

}  // namespace moeq
