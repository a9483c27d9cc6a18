"""Tensor-level wrappers over libmoeq.so.

Two groups:

* stage ops of the fused layer path (route, permute, grouped_gemm, combine,
  moe_forward), used by the QuantFused*MoEBlock modules and the tests;
* the reference's kernel-level operator surface with the same names minus
  the ``_triton`` suffix and the same argument meaning
  (gemq/triton_kernels/*.py): dequant_group_gemm, fused_dequant_up_proj,
  fused_dequant_down_proj, dequant_gemm, dequant_splitk_gemv,
  pack_weights_over_cols.  Like the reference kernels they read GemLite
  zeros, i.e. w = q * s + z' (gemq/triton_kernels/utils.py:206-210).

All launches go to torch's current stream; outputs are allocated with torch
(caching allocator), nothing synchronizes the host except the one-time
repacking of reference-layout tensors handed to the kernel-level operators.
"""

import weakref

import torch

from . import _lib as L
from .experts import QuantProjection, pack_codes, unpack_words


# ------------------------------------------------------------------ routing
def route(x, gate_w, top_k, norm_topk, logits=True, logit_bias=None):
    """Router of QuantFused*MoEBlock (gemq/inference/moe_block.py:790-797):
    returns (logits or None, idx int32 [T, k], w fp32 [T, k]).  An fp32
    gate_w reproduces DeepSeek's fp32 gate (moe_block.py:549)."""
    x = x.contiguous()
    T, H = x.shape
    E = gate_w.shape[0]
    dev = x.device
    gdt = L.dtype_code(gate_w.dtype)
    ldt = torch.float32 if gdt == L.F32 else x.dtype
    lg = torch.empty((T, E), dtype=ldt, device=dev) if logits else None
    idx = torch.empty((T, top_k), dtype=torch.int32, device=dev)
    w = torch.empty((T, top_k), dtype=torch.float32, device=dev)
    bias = None if logit_bias is None else logit_bias.float().contiguous()
    ws_bytes = 0 if logits else L.lib().moeq_route_workspace_size(T, E)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev) if ws_bytes else None
    L.check(L.lib().moeq_route(L.ptr(x), L.dtype_code(x.dtype), T, H, L.ptr(gate_w.contiguous()), gdt, L.ptr(bias),
                               E, top_k, int(bool(norm_topk)), L.ptr(lg), L.ptr(idx), L.ptr(w), L.ptr(ws), ws_bytes,
                               L.stream_handle(dev)),
            "moeq_route")
    return lg, idx, w


def route_from_logits(logits, top_k, norm_topk):
    logits = logits.contiguous()
    T, E = logits.shape
    dev = logits.device
    idx = torch.empty((T, top_k), dtype=torch.int32, device=dev)
    w = torch.empty((T, top_k), dtype=torch.float32, device=dev)
    L.check(L.lib().moeq_route_from_logits(L.ptr(logits), L.dtype_code(logits.dtype), T, E, top_k,
                                           int(bool(norm_topk)), L.ptr(idx), L.ptr(w), L.stream_handle(dev)),
            "moeq_route_from_logits")
    return idx, w


def permute(idx, n_experts, n_shared=0, bm=16):
    """Stable grouping (gemq/inference/moe_block.py:803-810) on the device.
    Returns a dict of device tensors (see moeq_permute in include/moeq.h)."""
    idx = idx.contiguous()
    T, k = idx.shape
    dev = idx.device
    lib = L.lib()
    Et = n_experts + n_shared
    max_tiles = lib.moeq_max_tiles(T, k, n_experts, n_shared, bm)
    ws_bytes = lib.moeq_permute_workspace_size(T, k, n_experts, n_shared)
    i32 = dict(dtype=torch.int32, device=dev)
    out = dict(
        counts=torch.empty(Et, **i32), offsets=torch.empty(Et + 1, **i32),
        row_token=torch.empty(T * k + n_shared * T, **i32), row_pair=torch.empty(T * k, **i32),
        inv_perm=torch.empty(T * k, **i32), tiles=torch.empty((max_tiles, 4), **i32),
        n_tiles=torch.empty(1, **i32), max_tiles=max_tiles, bm=bm)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    L.check(lib.moeq_permute(L.ptr(idx), T, k, n_experts, n_shared, bm, L.ptr(out["counts"]), L.ptr(out["offsets"]),
                             L.ptr(out["row_token"]), L.ptr(out["row_pair"]), L.ptr(out["inv_perm"]),
                             L.ptr(out["tiles"]), L.ptr(out["n_tiles"]), L.ptr(ws), ws_bytes, L.stream_handle(dev)),
            "moeq_permute")
    return out


# ------------------------------------------------------------- expert GEMMs
# Every row tile reads A through buffer loads with 32-bit byte offsets:
# every row it reads must end within the first 2 GiB of `a`.
A_ROWS_MAX_BYTES = 1 << 31


def a_rows_addressable(a, bm):
    """True when every row of `a` ends within the 2 GiB the tiles address
    (any tile class bm)."""
    return a.shape[0] * a.stride(0) * a.element_size() <= A_ROWS_MAX_BYTES


def grouped_gemm(a, rows, n_out, tiles, n_tiles, max_tiles, bm, p0, p1=None, row_src=None,
                 out_dtype=torch.float16, splits=1):
    """One launch over all row tiles: out[r] = A[row_src[r]] @ deq(W[expert(r)])
    (STORE), or silu(. @ W_p0) * (. @ W_p1) when p1 is given (SILU_MUL).
    Returns [rows, N] (or [splits, rows, N] fp32 for split-K)."""
    dev = a.device
    N = p0.N
    if a.dtype == torch.bfloat16 and bm >= 32:
        a = a.to(torch.float16)  # LDS-staged tiles read F16 rows (exact for |x| in fp16 range)
    if not a_rows_addressable(a, bm):
        raise ValueError(f"grouped_gemm: activations of {a.shape[0]} rows x {a.stride(0)} elements exceed "
                         f"{A_ROWS_MAX_BYTES} bytes (split the rows, as QuantLinear.forward does)")
    epi = L.EPI_SILU_MUL if p1 is not None else L.EPI_STORE
    shape = (rows, N) if splits == 1 else (splits, rows, N)
    out = torch.empty(shape, dtype=out_dtype, device=dev)
    g = L.MoeqGemm(a=a.data_ptr(), a_dtype=L.dtype_code(a.dtype), lda=a.stride(0),
                   row_src=row_src.data_ptr() if row_src is not None else None,
                   tiles=tiles.data_ptr(), n_tiles=n_tiles.data_ptr(), max_tiles=max_tiles, bm=bm,
                   epilogue=epi, out=out.data_ptr(), out_dtype=L.dtype_code(out_dtype), ldo=N, splits=splits,
                   split_stride=rows * N)
    s0 = p0.struct()
    s1 = p1.struct() if p1 is not None else None
    L.check(L.lib().moeq_grouped_gemm(g, s0, s1 if s1 is not None else None, L.stream_handle(dev)),
            "moeq_grouped_gemm")
    return out


def combine(y, inv_perm, w, T, top_k, n_shared, out_dtype):
    """Deterministic top-k weighted combine (gemq/inference/moe_block.py:811-812)."""
    dev = y.device
    splits = 1 if y.dim() == 2 else y.shape[0]
    rows, H = y.shape[-2], y.shape[-1]
    out = torch.empty((T, H), dtype=out_dtype, device=dev)
    L.check(L.lib().moeq_combine(L.ptr(y), L.dtype_code(y.dtype), splits, rows * H, H, L.ptr(inv_perm), L.ptr(w),
                                 T, top_k, n_shared, H, L.ptr(out), L.dtype_code(out_dtype), L.stream_handle(dev)),
            "moeq_combine")
    return out


# --------------------------------------------------------------- whole layer
class MoELayer:
    """Device weights of one MoE layer and the C descriptor pointing at them."""

    def __init__(self, gate_w, w1: QuantProjection, w3: QuantProjection, w2: QuantProjection,
                 top_k, norm_topk, act_dtype, n_shared=0, logit_bias=None, one_token_act_softmax=False):
        """one_token_act_softmax: forward(..., one_token=True) of a single
        token routes on softmax probabilities rounded to act_dtype and
        renormalises in act_dtype, as Mixtral's forward_one_token does
        (gemq/inference/moe_block.py:280-283); every other call ranks the
        logits with fp32 softmax weights."""
        E_total = w1.E
        self.n_shared = n_shared
        self.n_experts = E_total - n_shared
        assert gate_w.shape[0] == self.n_experts
        if w1.nbits_list != w3.nbits_list:
            raise ValueError("gate_proj and up_proj must share per-expert bit-widths "
                             "(gemq/inference/moe_block.py:69-80)")
        self.gate_w = gate_w.contiguous()
        self.w1, self.w3, self.w2 = w1, w3, w2
        self.hidden, self.inter = w1.K, w1.N
        self.top_k, self.norm_topk = int(top_k), bool(norm_topk)
        self.act_dtype = act_dtype
        self.logit_bias = None if logit_bias is None else logit_bias.float().contiguous()
        self.desc = L.MoeqMoe(
            hidden=self.hidden, inter=self.inter, n_experts=self.n_experts, top_k=self.top_k,
            n_shared=n_shared, act_dtype=L.dtype_code(act_dtype), gate_dtype=L.dtype_code(self.gate_w.dtype),
            norm_topk=int(self.norm_topk), gate_w=self.gate_w.data_ptr(),
            w1=w1.struct(), w3=w3.struct(), w2=w2.struct(),
            logit_bias=None if self.logit_bias is None else self.logit_bias.data_ptr())
        self.one_token_act_softmax = bool(one_token_act_softmax)
        self.desc_one_token = self.desc
        if self.one_token_act_softmax:
            self.desc_one_token = L.MoeqMoe.from_buffer_copy(self.desc)
            self.desc_one_token.one_token_act_softmax = 1
        self._ws = None

    def workspace_size(self, T):
        return L.lib().moeq_moe_workspace_size(self.desc, T)

    def plan(self, T):
        import ctypes
        buf = (ctypes.c_int32 * 4)()
        L.check(L.lib().moeq_moe_plan(self.desc, T, buf), "moeq_moe_plan")
        return dict(bm=buf[0], splits=buf[1], max_tiles=buf[2], y_dtype=buf[3])

    def workspace_layout(self, T):
        """Byte offsets in the forward's workspace of idx, w, counts, offsets,
        row_token, row_pair, inv_perm, tiles, n_tiles (for tests)."""
        import ctypes
        buf = (ctypes.c_int64 * 9)()
        L.check(L.lib().moeq_moe_workspace_layout(self.desc, T, buf), "moeq_moe_workspace_layout")
        return list(buf)

    def workspace(self, T, device):
        need = max(self.workspace_size(T), 1)
        if self._ws is None or self._ws.numel() < need or self._ws.device != device:
            self._ws = torch.empty(need, dtype=torch.uint8, device=device)
        return self._ws

    def forward(self, x, out_dtype=None, want_logits=True, out=None, logits=None, gate_up_events=None,
                one_token=False):
        """x [T, H] -> (out [T, H], logits [T, E] or None).  gate_up_events:
        optional pair of recorded torch.cuda.Event, re-recorded on the
        current stream just before and after the gate/up launch.  one_token:
        the call is a forward_one_token (selects the one-token routing of
        one_token_act_softmax layers)."""
        assert x.dim() == 2 and x.shape[1] == self.hidden, x.shape
        desc = self.desc_one_token if one_token else self.desc
        if x.dtype != self.act_dtype:
            raise TypeError(f"activations are {x.dtype}, layer expects {self.act_dtype}")
        x = x.contiguous()
        T = x.shape[0]
        dev = x.device
        odt = out_dtype or self.act_dtype
        if out is None:
            out = torch.empty((T, self.hidden), dtype=odt, device=dev)
        if want_logits and logits is None:
            ldt = torch.float32 if self.gate_w.dtype == torch.float32 else self.act_dtype
            logits = torch.empty((T, self.n_experts), dtype=ldt, device=dev)
        ws = self.workspace(T, dev)
        if gate_up_events is not None:
            e0, e1 = (e._as_parameter_ for e in gate_up_events)
            if not e0.value or not e1.value:
                raise ValueError("gate_up_events must have been recorded once (torch creates them lazily)")
            L.check(L.lib().moeq_moe_forward_timed(desc, L.ptr(x), T, L.ptr(out), L.dtype_code(odt),
                                                   L.ptr(logits) if want_logits else None, L.ptr(ws),
                                                   ws.numel(), L.stream_handle(dev), e0, e1),
                    "moeq_moe_forward_timed")
            return out, (logits if want_logits else None)
        L.check(L.lib().moeq_moe_forward(desc, L.ptr(x), T, L.ptr(out), L.dtype_code(odt),
                                         L.ptr(logits) if want_logits else None, L.ptr(ws), ws.numel(),
                                         L.stream_handle(dev)), "moeq_moe_forward")
        return out, (logits if want_logits else None)


# ------------------------------------------- reference kernel-level surface
# Build-layout projections derived from reference-stacked tensors, keyed on
# the identity of those tensors.  An entry holds weak references to them and
# their version counters: it is used only while every tensor is the same live,
# unmodified object (a new tensor can reuse a freed address or a dead
# object's id, but never a live weak reference), and is dropped as soon as
# one of them is freed.  Nothing here keeps the source tensors alive: the
# projection holds its own copies.
_REPACK_CACHE = {}


def _cached_proj(tensors, extra, build):
    key = tuple(id(t) for t in tensors) + tuple(extra)
    versions = tuple(t._version for t in tensors)
    hit = _REPACK_CACHE.get(key)
    if hit is not None:
        refs, vers, proj = hit
        if vers == versions and all(r() is t for r, t in zip(refs, tensors)):
            return proj
    proj = build()

    def drop(_ref, key=key):
        _REPACK_CACHE.pop(key, None)

    _REPACK_CACHE[key] = (tuple(weakref.ref(t, drop) for t in tensors), versions, proj)
    return proj


def _proj_from_stacked(wq, scales, zeros, nbits, wq_strides, zs_strides, K, group_size):
    """Build-layout view of reference-stacked tensors (GemLite zeros).  nbits,
    wq_strides and group_size may be tensors or Python ints; zs_strides None
    means the uniform scale offsets e * (K / g) * N the decode kernels assume
    (fused_dequant_bmm.py:62, :218).  Host reads of the meta tensors happen
    only when the projection is built, not per call."""
    src = [t for t in (wq, scales, zeros, nbits, wq_strides, zs_strides, group_size) if torch.is_tensor(t)]
    extra = (K,) + tuple(None if torch.is_tensor(t) else t for t in (nbits, wq_strides, zs_strides, group_size))

    def build():
        nb = [int(b) for b in nbits.tolist()] if torch.is_tensor(nbits) else [int(nbits)]
        gs = int(group_size.reshape(-1)[0].item()) if torch.is_tensor(group_size) else int(group_size)
        N = wq.shape[1]
        G = K // gs
        wst = [int(v) for v in wq_strides.tolist()] if torch.is_tensor(wq_strides) else [int(wq_strides)]
        zst = [int(v) for v in zs_strides.tolist()] if zs_strides is not None else [e * G * N for e in range(len(nb))]
        flat_w, flat_s, flat_z = wq.reshape(-1), scales.reshape(-1), zeros.reshape(-1)
        words, sc, ze = [], [], []
        for e, b in enumerate(nb):
            rows = -(-K // (32 // b))
            words.append(flat_w[wst[e]:wst[e] + rows * N].view(rows, N))
            sc.append(flat_s[zst[e]:zst[e] + G * N].view(G, N))
            ze.append(flat_z[zst[e]:zst[e] + G * N].view(G, N))
        return QuantProjection(words, sc, ze, nb, K, N, gs, L.DQ_AFFINE)

    return _cached_proj(src, extra, build)


def _bm_for(m):
    return 16 if m <= 16 else 32 if m <= 32 else 64 if m <= 64 else 128 if m < 192 else 256


def _slot_tiles(expert_ids, rows_per_slot, bm):
    """Row tiles for `A` slots of `rows_per_slot` rows each, slot a computed
    with expert expert_ids[a] (device tensor, no host sync)."""
    A = expert_ids.shape[0]
    nmt = -(-rows_per_slot // bm)
    dev = expert_ids.device
    a = torch.arange(A, device=dev).repeat_interleave(nmt)
    j = torch.arange(nmt, device=dev).repeat(A)
    r0 = a * rows_per_slot + j * bm
    rc = torch.clamp(rows_per_slot - j * bm, max=bm)
    tiles = torch.stack([expert_ids.to(torch.int64)[a], r0, rc, torch.zeros_like(rc)], dim=1).to(torch.int32)
    n = torch.full((1,), A * nmt, dtype=torch.int32, device=dev)
    return tiles.contiguous(), n, A * nmt


def silu_mul(x1, x3):
    """fp16(silu(x1) * x3) computed in fp32 (moeq_silu_mul), the prologue of
    fused_dequant_down_proj_triton (fused_dequant_bmm.py:236-239)."""
    assert x1.shape == x3.shape and x1.dtype == x3.dtype == torch.float16
    x1, x3 = x1.contiguous(), x3.contiguous()
    out = torch.empty_like(x1)
    L.check(L.lib().moeq_silu_mul(L.ptr(x1), L.ptr(x3), x1.numel(), L.ptr(out), L.stream_handle(x1.device)),
            "moeq_silu_mul")
    return out


def dequant_group_gemm(x, indices, wq, scales, zeros, nbits, group_sizes, wq_strides, zs_strides,
                       compute_dtype=torch.float16):
    """out[a] = x @ dequantize(wq[indices[a]]), [A, M, N] fp16.
    gemq/triton_kernels/dequant_group_gemm.py:155-202."""
    if compute_dtype != torch.float16:
        raise ValueError("dequant_group_gemm computes in float16 (as the reference)")
    M, K = x.shape
    N = wq.shape[1]
    A = indices.shape[0]
    proj = _proj_from_stacked(wq, scales, zeros, nbits, wq_strides, zs_strides, K, group_sizes)
    bm = _bm_for(M)
    tiles, n, mt = _slot_tiles(indices.reshape(-1), M, bm)
    row_src = torch.arange(A * M, device=x.device, dtype=torch.int32) % M
    out = grouped_gemm(x.contiguous(), A * M, N, tiles, n, mt, bm, proj, row_src=row_src)
    return out.view(A, M, N)


def fused_dequant_up_proj(x, idx, w1, w3, w1_scales, w1_zeros, w3_scales, w3_zeros, nbits, w_strides,
                          group_size):
    """(x1, x3) = (x @ deq(w1[idx[a]]), x @ deq(w3[idx[a]])) as [1, A*N] fp16.
    gemq/triton_kernels/fused_dequant_bmm.py:122-173 (w3 read at w1's
    offsets and bit-widths, scale offsets idx * K/g as the reference)."""
    _, K = x.shape
    N = w1.shape[1]
    A = idx.shape[0]
    p1 = _proj_from_stacked(w1, w1_scales, w1_zeros, nbits, w_strides, None, K, group_size)
    p3 = _proj_from_stacked(w3, w3_scales, w3_zeros, nbits, w_strides, None, K, group_size)
    tiles, n, mt = _slot_tiles(idx.reshape(-1), 1, 16)
    row_src = torch.zeros(A, dtype=torch.int32, device=x.device)
    xc = x.contiguous()
    x1 = grouped_gemm(xc, A, N, tiles, n, mt, 16, p1, row_src=row_src)
    x3 = grouped_gemm(xc, A, N, tiles, n, mt, 16, p3, row_src=row_src)
    return x1.view(1, A * N), x3.view(1, A * N)


def fused_dequant_down_proj(x1, x3, idx, w2, w2_scales, w2_zeros, nbits, w_strides, group_size):
    """x2[a] = (silu(x1[a]) * x3[a]) @ deq(w2[idx[a]]) as [1, A*N] fp16.
    gemq/triton_kernels/fused_dequant_bmm.py:264-312.  The fp32 SiLU*mul
    prologue (:236-239) runs as moeq_silu_mul, whose fp16 product the
    grouped GEMM reads."""
    A = idx.shape[0]
    K = x1.shape[1] // A
    N = w2.shape[1]
    h = silu_mul(x1, x3).view(A, K)
    p2 = _proj_from_stacked(w2, w2_scales, w2_zeros, nbits, w_strides, None, K, group_size)
    tiles, n, mt = _slot_tiles(idx.reshape(-1), 1, 16)
    out = grouped_gemm(h, A, N, tiles, n, mt, 16, p2)
    return out.view(1, A * N)


def dequant_gemm(x, w_q, scales, zeros, nbits, group_size):
    """x @ dequantize(w_q), [M, N] fp16.  gemq/triton_kernels/dequant_gemm.py:150-193."""
    M, K = x.shape
    proj = _proj_from_stacked(w_q, scales, zeros, int(nbits), 0, None, K, int(group_size))
    bm = _bm_for(M)
    one = torch.zeros(1, dtype=torch.int32, device=x.device)
    tiles, n, mt = _slot_tiles(one, M, bm)
    return grouped_gemm(x.contiguous(), M, w_q.shape[1], tiles, n, mt, bm, proj)


def dequant_splitk_gemv(x, w_q, scales, zeros, nbits, group_size):
    """x[1, K] @ dequantize(w_q) -> [1, N] fp16; deterministic (fixed-order
    reduction instead of the reference's fp16 atomics,
    gemq/triton_kernels/dequant_gemv.py:43-156)."""
    assert x.shape[0] == 1
    return dequant_gemm(x, w_q, scales, zeros, nbits, group_size)


def pack_weights_over_cols(W_q, W_nbits, packing_bitwidth=32, transpose=True):
    """gemq/triton_kernels/utils.py:74-113: uint8 codes [N, K] -> int32 words,
    [ceil(K/eps), N] when transpose (the default) else [N, ceil(K/eps)];
    returns (words, eps)."""
    assert packing_bitwidth == 32, "Unsuported bitpacking width"
    assert W_nbits in (4, 3, 2, 1), f"Untested quantization bitwidth: {W_nbits}"
    words = pack_codes(W_q.to(torch.uint8), int(W_nbits))
    return (words if transpose else words.t()), 32 // int(W_nbits)


__all__ = [
    "route", "route_from_logits", "permute", "grouped_gemm", "combine", "MoELayer",
    "silu_mul", "dequant_group_gemm", "fused_dequant_up_proj", "fused_dequant_down_proj", "dequant_gemm",
    "dequant_splitk_gemv", "pack_weights_over_cols", "unpack_words",
]
