"""Quantized expert projections: the reference's stacked tensors plus the
build layout the HIP kernels read.

QuantFused*MoEBlock.from_hf (gemq/inference/moe_block.py:725-757) concatenates
each expert's GemLite tensors into
    wq      [sum_e ceil(K/eps_e), N] int32     (packed codes, N contiguous)
    scales  [sum_e K/g, N] fp16
    zeros   [sum_e K/g, N] fp16
and builds int32 [E] meta tensors nbits, group_sizes and the exclusive
cumsums wq_strides / zs_strides.  QuantProjection keeps exactly those (so code
that pokes the attributes keeps working) and, once at load time, derives
    words    build-layout codes (moeq_repack, panel-major), word_off [E] int64
    sz       fused (scale, zero) half2 pairs (moeq_prep_scales, panel-major),
             sz_off [E]
"""

import ctypes

import torch

from . import _lib as L


def _excl_cumsum(values):
    out, run = [], 0
    for v in values:
        out.append(run)
        run += v
    return out


def pack_codes(codes: torch.Tensor, nbits: int) -> torch.Tensor:
    """uint8 codes [N, K] (device) -> reference-layout int32 words
    [ceil(K/eps), N] via moeq_pack_cols (gemq/triton_kernels/utils.py:74-113)."""
    assert codes.dtype == torch.uint8 and codes.is_cuda and codes.dim() == 2
    codes = codes.contiguous()
    N, K = codes.shape
    eps = 32 // nbits
    out = torch.empty((-(-K // eps), N), dtype=torch.int32, device=codes.device)
    L.check(L.lib().moeq_pack_cols(L.ptr(codes), N, K, nbits, L.ptr(out), L.stream_handle(codes.device)),
            "moeq_pack_cols")
    return out


def unpack_words(words: torch.Tensor, nbits: int, K: int) -> torch.Tensor:
    """Reference-layout words [rows, N] -> uint8 codes [N, K] (load time; the
    read pattern of gemq/triton_kernels/dequant_group_gemm.py:118-130)."""
    eps = 32 // nbits
    k = torch.arange(K, device=words.device)
    w = words[k // eps, :].to(torch.int64) & 0xFFFFFFFF
    sh = ((k % eps) * nbits).to(torch.int64)[:, None]
    return ((w >> sh) & ((1 << nbits) - 1)).to(torch.uint8).t().contiguous()


class QuantProjection:
    """One projection (gate_proj, up_proj or down_proj) of all experts.

    ref_words[e]: int32 [ceil(K/eps_e), N]; scales[e] / zeros[e]: fp16
    [K/g, N]; nbits[e]: int.  dq_mode: L.DQ_HQQ when zeros are HQQ zero points
    (w = (q - z) * s), L.DQ_AFFINE when they are GemLite's z' = -z*s
    (w = q * s + z')."""

    def __init__(self, ref_words, scales, zeros, nbits, K, N, group_size, dq_mode):
        E = len(ref_words)
        assert len(scales) == len(zeros) == len(nbits) == E and E > 0
        if K % 128 or N % 16 or group_size % 32 or K % group_size:
            raise ValueError(f"unsupported projection K={K} N={N} group_size={group_size} "
                             "(needs K % 128 == 0, N % 16 == 0, group_size a multiple of 32 dividing K)")
        for b in nbits:
            if b not in (1, 2, 3, 4):
                raise ValueError(f"nbits={b} not in 1..4")
        dev = ref_words[0].device
        self.K, self.N, self.group_size, self.dq_mode, self.E = K, N, group_size, dq_mode, E
        self.nbits_list = [int(b) for b in nbits]
        # reference attribute set (moe_block.py:725-757)
        self.wq = torch.cat([w.contiguous() for w in ref_words])
        self.scales = torch.cat([s.contiguous() for s in scales]).to(torch.float16)
        self.zeros = torch.cat([z.contiguous() for z in zeros]).to(torch.float16)
        self.nbits = torch.tensor(self.nbits_list, dtype=torch.int32, device=dev)
        self.group_sizes = torch.full((E,), group_size, dtype=torch.int32, device=dev)
        self.wq_strides = torch.tensor(_excl_cumsum([w.numel() for w in ref_words]), dtype=torch.int32, device=dev)
        self.zs_strides = torch.tensor(_excl_cumsum([s.numel() for s in scales]), dtype=torch.int32, device=dev)
        # build layout
        sizes = [K * N * b // 32 for b in self.nbits_list]
        offs = _excl_cumsum(sizes)
        self.words = torch.empty(sum(sizes), dtype=torch.int32, device=dev)
        st = L.stream_handle(dev)
        lib = L.lib()
        for e in range(E):
            dst = self.words[offs[e]:offs[e] + sizes[e]]
            L.check(lib.moeq_repack(L.ptr(ref_words[e].contiguous()), K, N, self.nbits_list[e], L.ptr(dst), st),
                    "moeq_repack")
        self.word_off = torch.tensor(offs, dtype=torch.int64, device=dev)
        if dq_mode == L.DQ_HQQ:
            z = self.zeros
            if bool(((z == torch.round(z)) & (z >= 0) & (z <= 1023)).all()):
                # integer zero points: one fp16 op less per weight pair, same weights
                dq_mode = L.DQ_HQQ_INT
        self.dq_mode = dq_mode
        G = K // group_size
        self.sz = torch.empty(E * G * N, dtype=torch.int32, device=dev)
        L.check(lib.moeq_prep_scales(L.ptr(self.scales), L.ptr(self.zeros), E, G, N, dq_mode,
                                     L.ptr(self.sz), st), "moeq_prep_scales")
        self.sz_off = torch.tensor(_excl_cumsum([s.numel() for s in scales]), dtype=torch.int64, device=dev)

    @classmethod
    def from_triplets(cls, triplets):
        """From HQQ logical triplets (robustgemq_amd.quantize.QuantTriplet),
        one per expert, all on the same CUDA device."""
        N, K = triplets[0].shape
        g = triplets[0].group_size
        words, sc, ze, nb = [], [], [], []
        for t in triplets:
            assert t.shape == (N, K) and t.group_size == g
            words.append(pack_codes(t.codes(), t.nbits))
            sc.append(t.scales_nk().half())
            ze.append(t.zeros_nk().half())
            nb.append(t.nbits)
        return cls(words, sc, ze, nb, K, N, g, L.DQ_HQQ)

    def struct(self):
        return L.MoeqProj(
            words=self.words.data_ptr(), word_off=self.word_off.data_ptr(),
            sz=self.sz.data_ptr(), sz_off=self.sz_off.data_ptr(), nbits=self.nbits.data_ptr(),
            K=self.K, N=self.N, group_size=self.group_size, dq_mode=self.dq_mode)

    def weight_bytes(self, experts=None):
        """Algorithmic bytes of the packed codes plus fp16 scale and zero of
        the given experts (all by default): ceil(K/eps)*N*4 + 4*N*K/g each."""
        ids = range(self.E) if experts is None else experts
        tot = 0
        for e in ids:
            b = self.nbits_list[e]
            tot += -(-self.K // (32 // b)) * self.N * 4 + 4 * self.N * self.K // self.group_size
        return tot
