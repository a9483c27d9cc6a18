"""Routing and token->expert permutation (CPU restatement).

Reference: gemq/inference/moe_block.py
  :790-797   router_logits = gate(x); softmax(fp32); topk; optional renorm
  :243-249   Mixtral (always renormalized)
  :549-556   DeepSeek (fp32 gate: F.linear(x.float(), W.float()))
  :803-810   one_hot(...).permute(2,1,0) -> [E, k, T]; expert_hit; torch.where
"""

import ctypes
import os

import numpy as np

from .fp import near_midpoint, round_to

_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(os.path.dirname(__file__), "_build", "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle C library missing: {path} (run make -C oracle)")
        lib = ctypes.CDLL(path)
        lib.oracle_router_logits.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                             ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
        lib.oracle_router_logits.restype = None
        _LIB = lib
    return _LIB


def router_logits_fixed(x32, w32):
    """fp32 x[T, H] @ w[E, H]^T in the pinned order of router_exact.c."""
    x32 = np.ascontiguousarray(x32, dtype=np.float32)
    w32 = np.ascontiguousarray(w32, dtype=np.float32)
    T, H = x32.shape
    E = w32.shape[0]
    out = np.empty((T, E), np.float32)
    _lib().oracle_router_logits(x32.ctypes.data, w32.ctypes.data, T, H, E, out.ctypes.data)
    return out


def router_logits(x32, w32, logits_dtype, bias=None):
    """Router logits as the reference exposes them: computed in fp32 and
    rounded to the gate's output dtype ('f16' / 'bf16'; 'f32' for DeepSeek's
    fp32 gate, moe_block.py:549).  ``bias`` (fp32 [E], optional) is a routing
    prior added in fp32 before rounding (synthetic skewed workloads only; the
    reference has none).  Returned as fp32 values."""
    lg = router_logits_fixed(x32, w32)
    if bias is not None:
        lg = (lg + np.asarray(bias, dtype=np.float32)[None, :]).astype(np.float32)
    return round_to(lg, logits_dtype)


def topk_route(logits32, top_k, norm_topk):
    """softmax(fp32) -> topk -> renorm, moe_block.py:792-795.

    Ranking is by logit (softmax is monotone), ties resolved towards the lower
    expert index.  Returns (idx int32 [T, k], w fp32 [T, k]) with the slots in
    descending order of probability, as torch.topk returns them."""
    lg = np.asarray(logits32, dtype=np.float32)
    T, E = lg.shape
    idx = np.argsort(-lg, axis=1, kind="stable")[:, :top_k].astype(np.int32)
    m = lg.max(axis=1, keepdims=True)
    e = np.exp((lg - m).astype(np.float64))
    p = (e / e.sum(axis=1, keepdims=True)).astype(np.float32)
    w = np.take_along_axis(p, idx.astype(np.int64), axis=1)
    if norm_topk:
        w = (w.astype(np.float64) / w.astype(np.float64).sum(axis=1, keepdims=True)).astype(np.float32)
    return idx, w


def topk_route_act_softmax(logits32, top_k, dtype):
    """Mixtral's forward_one_token router, moe_block.py:280-283:

        expert_weights = F.softmax(scores, dim=-1)          # scores in `dtype`
        expert_weights, expert_indices = torch.topk(expert_weights, top_k)
        expert_weights /= expert_weights.sum(dim=-1, keepdim=True)

    torch runs softmax on a 16-bit tensor in fp32 and rounds each output to
    the tensor's type; topk ranks those rounded values (equal values: the
    lower expert index first, the order the kernels use; CUDA's tie order is
    not specified); the sum accumulates in fp32 and is rounded, and so is
    each quotient.  dtype: 'f16' | 'bf16'.  Returns (idx int32 [T, k], w fp32
    [T, k] holding `dtype` values, p fp32 [T, E] the rounded probabilities,
    fragile bool [T] marking tokens with a probability within a few fp32 ulps
    of a rounding midpoint of `dtype`: any fp32 softmax, torch's included,
    may round those to the other neighbour)."""
    lg = np.asarray(logits32, dtype=np.float32)
    m = lg.max(axis=1, keepdims=True)
    e = np.exp((lg - m).astype(np.float64))
    p32 = (e / e.sum(axis=1, keepdims=True)).astype(np.float32)
    p = round_to(p32, dtype)
    idx = np.argsort(-p, axis=1, kind="stable")[:, :top_k].astype(np.int32)
    sel = np.take_along_axis(p, idx.astype(np.int64), axis=1)
    s = round_to(sel.sum(axis=1, keepdims=True, dtype=np.float32), dtype)
    w = round_to((sel / s).astype(np.float32), dtype)
    return idx, w, p, near_midpoint(p32, dtype).any(axis=1)


def permute(idx, n_experts, n_shared=0):
    """Token->expert grouping in the reference order (moe_block.py:803-810):
    experts ascending; within an expert, torch.where over the [k, T] mask gives
    (slot, token) ascending.  That is a stable sort by expert of the slot-major
    flattening of idx.

    Returns dict with counts, offsets, row_token, row_pair (t*k + slot),
    inv_perm; shared experts append T rows each (token order)."""
    idx = np.asarray(idx, dtype=np.int64)
    T, k = idx.shape
    seq = idx.T.reshape(-1)  # position p = slot*T + t
    order = np.argsort(seq, kind="stable")
    slot = order // T
    tok = order % T
    row_pair = (tok * k + slot).astype(np.int32)
    inv_perm = np.empty(T * k, np.int32)
    inv_perm[row_pair] = np.arange(T * k, dtype=np.int32)
    counts = np.bincount(seq, minlength=n_experts).astype(np.int32)
    counts = np.concatenate([counts, np.full(n_shared, T, np.int32)])
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    row_token = np.concatenate([tok, np.tile(np.arange(T), n_shared)]).astype(np.int32)
    return dict(counts=counts, offsets=offsets, row_token=row_token,
                row_pair=row_pair, inv_perm=inv_perm)


def permute_loop(idx, n_experts):
    """The same grouping written as the reference's loop: for each hit expert
    ascending, torch.where(expert_mask[e]) over the [k, T] mask (row-major:
    slot outer, token inner).  Used to pin ``permute``."""
    idx = np.asarray(idx)
    T, k = idx.shape
    rows = []
    for e in range(n_experts):
        for s in range(k):
            for t in range(T):
                if idx[t, s] == e:
                    rows.append(t * k + s)
    return np.array(rows, np.int32)
