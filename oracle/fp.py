"""IEEE half / bfloat16 element-wise arithmetic the way torch evaluates it.

torch computes every fp16 / bf16 element-wise op in fp32 ("opmath") and rounds
the result to the storage type with round-to-nearest-even, on CPU and GPU
alike.  The reference's fake-quant weights ``((Q - zeros) * scales)``
(gemq/quantizers/rtn.py:57-61) and its RTN quantizer (rtn.py:42-53) are
sequences of such ops, so they are restated here op by op.  numpy's own
float16 loops are not relied on (they may use native fp16 instructions on
some hosts, which round once instead of twice).
"""

import numpy as np

F16 = np.float16
F32 = np.float32


def f32(a):
    return np.asarray(a).astype(np.float32)


def to_f16(a32):
    """fp32 -> fp16, round to nearest even (numpy's cast is IEEE RNE)."""
    return np.asarray(a32, dtype=np.float32).astype(np.float16)


def h_add(a, b):
    return to_f16(f32(a) + f32(b))


def h_sub(a, b):
    return to_f16(f32(a) - f32(b))


def h_mul(a, b):
    return to_f16(f32(a) * f32(b))


def h_div(a, b):
    return to_f16(f32(a) / f32(b))


def to_bf16_bits(a32):
    """fp32 -> bf16 bit pattern (uint16), round to nearest even; NaN kept quiet."""
    u = np.asarray(a32, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_to_bf16(a32):
    """fp32 values rounded to the nearest bf16, returned as fp32."""
    return bf16_bits_to_f32(to_bf16_bits(a32))


def near_midpoint(a32, dtype, ulps=4):
    """True where a positive fp32 value lies within `ulps` fp32 ulps of a
    rounding midpoint of `dtype` ('f16' normal range | 'bf16'): there two fp32
    evaluations of the same formula that differ in their last bits may round
    to different neighbours."""
    u = np.asarray(a32, dtype=np.float32).view(np.uint32).astype(np.int64)
    if dtype == "bf16":
        low, mid = u & 0xFFFF, 0x8000
    elif dtype == "f16":
        low, mid = u & 0x1FFF, 0x1000
    else:
        return np.zeros(u.shape, bool)
    return np.abs(low - mid) <= ulps


def round_to(a32, dtype):
    """Round fp32 values to the storage dtype name ('f16' | 'bf16' | 'f32'),
    returned as fp32 values."""
    if dtype == "f16":
        return to_f16(a32).astype(np.float32)
    if dtype == "bf16":
        return round_to_bf16(a32)
    if dtype == "f32":
        return np.asarray(a32, dtype=np.float32)
    raise ValueError(dtype)
