"""The per-expert dequantize-then-matmul loop in fp32 (the "fp32 reference").

Restates QuantFused*MoEBlock.forward_n_tokens with dense fake-quant weights:
  gemq/inference/moe_block.py:781-815   OLMoE (Qwen3 :1011-1045, Mixtral :234-267)
  gemq/inference/moe_block.py:540-578   DeepSeek, shared experts added unweighted (:575)
  gemq/inference/moe_block.py:763-779   forward_single_expert: x1=x@W1, x3=x@W3, (silu(x1)*x3)@W2
  gemq/triton_kernels/fused_dequant_bmm.py:236-239  SiLU in fp32
All arithmetic is fp32 (numpy BLAS); the reference's fp16 intermediate roundings
are deliberately absent, which is what "fp32 reference" means in the tests.
"""

import numpy as np

from .quant import dequant_hqq, dequant_affine
from .route import permute, router_logits, topk_route


def silu(v):
    v = np.asarray(v, dtype=np.float32)
    return v / (np.float32(1.0) + np.exp(-v))


def dense_weight(Q, s, z, N, K, dq_mode=0):
    """fp16 fake-quant weight [N, K] (out_features, in_features) from the HQQ
    triplet Q [N*K/g, g], s/z [N*K/g, 1] (tests/conftest.py:128-131)."""
    W = dequant_hqq(Q, s, z) if dq_mode == 0 else dequant_affine(Q, s, z)
    return W.reshape(N, K)


def expert_mlp(x32, W1, W3, W2):
    """forward_single_expert, moe_block.py:763-779, fp32.  W1/W3 [F, H], W2 [H, F]."""
    g = x32 @ W1.T
    u = x32 @ W3.T
    return (silu(g) * u) @ W2.T


def moe_from_routing(x32, idx, w, W1, W3, W2, shared=()):
    """Combine as forward_n_tokens does (moe_block.py:803-812), in fp32:
    experts ascending, rows in (slot, token) order, weighted index_add.
    W1/W3/W2: lists (per expert) of fp32 dense weights; shared: list of
    (W1, W3, W2) added with weight one (moe_block.py:575)."""
    T, H = x32.shape
    out = np.zeros((T, H), np.float32)
    E = len(W1)
    perm = permute(idx, E)
    for e in range(E):
        lo, hi = perm["offsets"][e], perm["offsets"][e + 1]
        if hi == lo:
            continue
        pairs = perm["row_pair"][lo:hi]
        tok, slot = pairs // idx.shape[1], pairs % idx.shape[1]
        y = expert_mlp(x32[tok], W1[e], W3[e], W2[e])
        np.add.at(out, tok, w[tok, slot][:, None] * y)
    for (S1, S3, S2) in shared:
        out += expert_mlp(x32, S1, S3, S2)
    return out


def moe_forward(x32, gate_w32, logits_dtype, top_k, norm_topk, W1, W3, W2, shared=(), bias=None):
    """Full layer: fixed-order router logits (rounded to the gate output
    dtype), top-k routing, expert loop.  Returns (out fp32 [T, H], logits fp32
    [T, E], idx, w)."""
    logits = router_logits(x32, gate_w32, logits_dtype, bias)
    idx, w = topk_route(logits, top_k, norm_topk)
    out = moe_from_routing(x32, idx, w, W1, W3, W2, shared)
    return out, logits, idx, w


def moe_dense_einsum(x32, idx, w, W1, W3, W2):
    """The dense formulation of the reference's Fused*MoEBlock.forward
    (moe_block.py:662-685): gather per-token expert weights, einsum, weighted
    sum.  A second formulation used to pin moe_from_routing."""
    W1s, W3s, W2s = np.stack(W1), np.stack(W3), np.stack(W2)
    w1 = W1s[idx]  # [T, A, F, H]
    w3 = W3s[idx]
    w2 = W2s[idx]  # [T, A, H, F]
    x1 = silu(np.einsum("ti,taoi->tao", x32, w1))
    x3 = np.einsum("ti,taoi->tao", x32, w3)
    eo = np.einsum("tao,taio->tai", x1 * x3, w2)
    return np.einsum("tai,ta->ti", eo, w)
