// 16-row grouped GEMM launches, fp32-output (split-K) kernels.
#include "gemm_bm16_impl.h"

namespace moeq {

template int launch16<MOEQ_F16, MOEQ_F32, false>(const GemmArgs &, int, int, hipStream_t);
template int launch16<MOEQ_BF16, MOEQ_F32, false>(const GemmArgs &, int, int, hipStream_t);

}  // namespace moeq
