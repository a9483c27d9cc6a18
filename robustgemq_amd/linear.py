"""Dense quantized linear: the E = 1 case of the grouped expert GEMM.

The reference keeps its attention and dense layers as GemLite linears built
from HQQ linears (create_gemlite_from_hqq, gemq/inference/patch.py:27-72;
replace_linear_recursive, :75-83).  QuantLinear takes the same inputs -- HQQ
codes [N, K] quantized along K with group g, scales and zero points
[N*K/g, 1], an optional bias -- and runs y = x @ W^T + b through
moeq_grouped_gemm with one expert: the 16-row decode tiles for up to 16
tokens, the LDS-staged MFMA tiles above.  The weight is the fake-quant weight
(Q - z) * s bit for bit, as the expert projections are.

For code that reads GemLite attributes (QuantFused*MoEBlock.from_hf reads
W_q, scales, zeros, W_nbits, group_size of each expert linear,
moe_block.py:720-733), the module also carries them in GemLite's convention:
W_q the packed words [ceil(K/eps), N], scales [K/g, N] and zeros
z' = -z * s [K/g, N].
"""

import torch
import torch.nn as nn

from . import _lib as L
from . import ops
from .experts import QuantProjection, pack_codes
from .quantize import QuantTriplet


def _bm_for_rows(m):
    return 16 if m <= 16 else 32 if m <= 32 else 64 if m <= 64 else 128


# Largest 16-row block count of a tile class and the next lower count the
# grouped GEMM has a variant for (tile_rows / tile_blocks_below in csrc/common.h).
_BLOCKS = {16: (2, 1), 32: (3, 2), 64: (6, 4), 128: (10, 8), 256: (16, 10)}


def split_rows(m, bm):
    """(row_start, row_count) of the tiles one expert's m rows take in class
    bm, cut as the device schedule of moeq_permute cuts them: ceil(m / cap)
    tiles at 16-row boundaries, the first x holding the largest block count
    and the rest the next lower one, x the fewest that hold every block."""
    smax, s2 = _BLOCKS[bm]
    B = -(-m // 16)
    nt = -(-B // smax)
    x = nt if smax == s2 else min(nt, max(0, -(-(B - s2 * nt) // (smax - s2))))
    out, b0 = [], 0
    for j in range(nt):
        b1 = min(b0 + (smax if j < x else s2), B)
        out.append((16 * b0, min(16 * b1, m) - 16 * b0))
        b0 = b1
    return out


class QuantLinear(nn.Module):
    """y = x @ dequant(W)^T (+ bias) for x [..., in_features]."""

    def __init__(self, codes, scales, zeros, nbits, group_size, bias=None, act_dtype=torch.float16):
        """codes: uint8 [N, K] on the GPU; scales, zeros: [N*K/g, 1] (HQQ
        layout, any float dtype; stored as fp16)."""
        super().__init__()
        assert codes.dim() == 2 and codes.is_cuda
        N, K = codes.shape
        g = int(group_size)
        if K % g:
            raise ValueError(f"in_features={K} is not a multiple of group_size={g}")
        self.in_features, self.out_features = K, N
        self.W_nbits, self.group_size = int(nbits), g
        self.act_dtype = act_dtype
        s_kn = scales.reshape(N, K // g).t().contiguous().to(torch.float16)
        z_kn = zeros.reshape(N, K // g).t().contiguous().to(torch.float16)
        words = pack_codes(codes.to(torch.uint8), self.W_nbits)
        self._proj = QuantProjection([words], [s_kn], [z_kn], [self.W_nbits], K, N, g, L.DQ_HQQ)
        # GemLite-convention views (what from_hf and the reference tests read)
        self.W_q = words
        self.scales = s_kn
        self.zeros = (-(z_kn.float() * s_kn.float())).to(torch.float16)
        self.bias = None if bias is None else bias.detach().to(device=codes.device, dtype=act_dtype).contiguous()
        self._tiles = {}

    # -- construction -------------------------------------------------------
    @classmethod
    def from_triplet(cls, t: QuantTriplet, bias=None, act_dtype=torch.float16):
        return cls(t.codes(), t.scales, t.zeros, t.nbits, t.group_size, bias=bias, act_dtype=act_dtype)

    @classmethod
    def from_hqq_layer(cls, hqq_layer, device=None, dtype=None):
        """The reads create_gemlite_from_hqq makes (patch.py:27-50): meta
        shape / nbits / group_size / axis / scale / zero, the codes from
        unpack(reshape=False, dtype=uint8) with the 3-bit padding rows cut
        (patch.py:37-39), and the bias."""
        meta = hqq_layer.meta
        out_features, in_features = meta["shape"]
        nbits, group_size = int(meta["nbits"]), int(meta["group_size"])
        assert meta["axis"] == 1, "Only axis==1 is supported."
        device = device or hqq_layer.W_q.device
        W_q = hqq_layer.unpack(reshape=False, dtype=torch.uint8)
        if nbits == 3:
            W_q = W_q[:out_features * in_features // group_size]
        W_q = W_q.reshape(out_features, in_features).to(device)
        scales, zeros = meta["scale"], meta["zero"]
        dtype = dtype or scales.dtype
        assert scales.dtype in (torch.float16, torch.bfloat16, torch.float32), \
            "Invalid scales.dtype, should floating point."
        bias = getattr(hqq_layer, "bias", None)
        return cls(W_q, scales.to(device), zeros.to(device), nbits, group_size, bias=bias,
                   act_dtype=dtype if dtype != torch.float32 else torch.float16)

    # -- forward ------------------------------------------------------------
    def _tile_list(self, M, dev):
        """Rows 0..M-1 of the single expert in tiles of at most
        moeq_tile_rows(bm) rows, cut as moeq_permute cuts an expert."""
        key = (M, dev)
        if key not in self._tiles:
            bm = _bm_for_rows(M)
            tiles = [(0, r0, rc, 0) for r0, rc in split_rows(M, bm)]
            nt = len(tiles)
            self._tiles[key] = (bm, torch.tensor(tiles, dtype=torch.int32, device=dev),
                                torch.tensor([nt], dtype=torch.int32, device=dev), nt)
        return self._tiles[key]

    def _gemm(self, x2):
        M = x2.shape[0]
        bm, tiles, n, nt = self._tile_list(M, x2.device)
        return ops.grouped_gemm(x2, M, self.out_features, tiles, n, nt, bm, self._proj)

    def forward(self, x):
        K = self.in_features
        assert x.shape[-1] == K, (x.shape, K)
        lead = x.shape[:-1]
        x2 = x.reshape(-1, K)
        if x2.dtype not in (torch.float16, torch.bfloat16):
            x2 = x2.to(self.act_dtype)
        x2 = x2.contiguous()
        M = x2.shape[0]
        if M == 0:
            return x.new_empty((*lead, self.out_features))
        # the tiles address rows with 32-bit offsets: run the rows in slices
        # that each stay within 2 GiB
        rows_max = max(16, (ops.A_ROWS_MAX_BYTES // (K * 2)) // 16 * 16)
        if M > rows_max:
            y = torch.cat([self._gemm(x2[r:r + rows_max]) for r in range(0, M, rows_max)])
        else:
            y = self._gemm(x2)
        y = y.to(x2.dtype)
        if self.bias is not None:
            y = y + self.bias.to(y.dtype)
        return y.reshape(*lead, self.out_features)

    def extra_repr(self):
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"nbits={self.W_nbits}, group_size={self.group_size}, bias={self.bias is not None}")


def replace_linear_recursive(module, make):
    """Replace every child for which make(child) returns a module
    (patch.py:75-83 replaces HQQLinear children with GemLite linears; here
    `make` decides, e.g. lambda m: QuantLinear.from_hqq_layer(m) if
    hasattr(m, "meta") else None)."""
    for name, child in module.named_children():
        new = make(child)
        if new is not None:
            setattr(module, name, new)
        else:
            replace_linear_recursive(child, make)
    return module


__all__ = ["QuantLinear", "replace_linear_recursive"]
