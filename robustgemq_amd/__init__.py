"""MI355X-native real-quant MoE expert path (routing, token grouping, mixed
1/2/3/4-bit grouped GEMM, fused SiLU*mul, weighted combine) behind the
QuantFused*MoEBlock interface of lcj1111/RobustGEMQ
(gemq/inference/moe_block.py).  Kernels: csrc/*.hip -> libmoeq.so (C ABI,
include/moeq.h), loaded with ctypes by _lib.py."""

__version__ = "0.1.0"
