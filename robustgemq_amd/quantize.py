"""Round-to-nearest group quantizer producing HQQ logical triplets.

Restates RTNWeightQuantizer.quantize (gemq/quantizers/rtn.py:15-55), the
weight source of the reference's synthetic tests (tests/conftest.py:117-131),
with torch fp16 tensors on any device.  Each step is one fp16 element-wise op
(torch evaluates it in fp32 and rounds), matching the reference op for op; the
divisors are tensors, so CPU and GPU both divide exactly (no reciprocal
multiply for scalar divisors).

The triplet layout is HQQ's axis=1 grouping (gemq/utils/quant_utils.py:55-98):
Q [N*K/g, g] codes, scales / zeros [N*K/g, 1], groups running along the input
dimension of a [N, K] (out_features, in_features) weight.
"""

from dataclasses import dataclass

import torch


@dataclass
class QuantTriplet:
    """One quantized linear: HQQ logical layout plus its shape."""
    Q: torch.Tensor       # [N*K/g, g] fp16 codes (integers 0 .. 2^b-1)
    scales: torch.Tensor  # [N*K/g, 1] fp16
    zeros: torch.Tensor   # [N*K/g, 1] fp16
    nbits: int
    group_size: int
    shape: tuple          # (N, K) = (out_features, in_features)

    def codes(self):
        """uint8 codes [N, K]."""
        N, K = self.shape
        return self.Q.reshape(N, K).to(torch.uint8)

    def scales_nk(self):
        """scales as [K/g, N] (the reference's stacked scale layout)."""
        N, K = self.shape
        return self.scales.reshape(N, K // self.group_size).t().contiguous()

    def zeros_nk(self):
        N, K = self.shape
        return self.zeros.reshape(N, K // self.group_size).t().contiguous()

    def dequantize(self):
        """Fake-quant weight ((Q - z) * s) in fp16, [N, K] (rtn.py:57-61)."""
        return ((self.Q - self.zeros) * self.scales).reshape(self.shape)

    def to(self, device):
        return QuantTriplet(self.Q.to(device), self.scales.to(device), self.zeros.to(device),
                            self.nbits, self.group_size, self.shape)


def rtn_quantize(W: torch.Tensor, nbits: int, group_size: int) -> QuantTriplet:
    """RTN min/max quantization of an fp16 weight [N, K] along K
    (gemq/quantizers/rtn.py:15-55).  The 1-bit scale 2*mean|W| (rtn.py:38) is
    an exact float64 sum / g, rounded to fp32 then fp16."""
    assert W.dtype == torch.float16, W.dtype
    N, K = W.shape
    assert K % group_size == 0, (K, group_size)
    Wg = W.reshape(-1, group_size)
    G = Wg.shape[0]
    dev = W.device
    if nbits == 1:  # rtn.py:36-40
        Q = (Wg >= 0).to(torch.float16)
        mean = Wg.abs().double().sum(dim=1, keepdim=True) / group_size
        s = mean.float().half() * 2
        z = torch.full((G, 1), 0.5, dtype=torch.float16, device=dev)
        return QuantTriplet(Q, s, z, nbits, group_size, (N, K))
    if nbits not in (2, 3, 4, 5, 6, 7, 8):
        raise ValueError(f"nbits={nbits}")
    mx = Wg.amax(dim=1, keepdim=True)
    mn = Wg.amin(dim=1, keepdim=True)
    max_int = 2 ** nbits - 1
    div = torch.full((1, 1), float(max_int), dtype=torch.float16, device=dev)
    floor = torch.full((1, 1), 1e-5, dtype=torch.float16, device=dev)
    s = torch.maximum(mx - mn, floor) / div  # rtn.py:47
    z = (-torch.round(mn / s)).clamp_(0, max_int)  # rtn.py:48
    Q = torch.clamp(torch.round(Wg / s) + z, 0, max_int)  # rtn.py:53
    return QuantTriplet(Q, s, z, nbits, group_size, (N, K))
