"""Writes tests/golden/golden.npz: small input / expected-output vectors of the
real-quant MoE path, computed by the pinned CPU oracle.

The reference commits no golden vectors (its tests draw inputs live with
CUDA-seeded torch RNG), so these are this build's own.  Inputs come from
numpy's PCG64 generator, which yields the same bits on every platform, so the
tests can regenerate the larger inputs (the layer weights) from their seed
and check them against the stored SHA-256 instead of storing them.

Contents (all arrays little-endian):
  rtn_b{1..4}_*      RTN quantizer (gemq/quantizers/rtn.py:15-55) on an fp16
                     [8, 256] weight with g = 64, one constant group included
  pack_b{1..4}_*     reference word packing (gemq/triton_kernels/utils.py:74-113)
                     of uint8 codes [16, 320] and the build layout of [:, :256]
  route_*            router logits (fp16, bit patterns), top-k with and without
                     renormalisation, the token->expert permutation, for
                     x [16, 512] fp16 and an fp16 gate [8, 512], k = 2
  route32_*          fp32 gate [16, 512] (DeepSeek style), k = 6, 2 shared experts
  block_*            one MoE layer at the reference's block-test shape
                     (tests/test_moe_block_equiv.py:29-38: H = F = 512, E = 8,
                     k = 2, g = 128, bits [1,2,3,2,3,1,2,3]), T = 16: logits,
                     routing, fp32 output of the dequantize-then-matmul loop

Run from the repository root:  python tests/golden/make_golden.py
"""

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import moe as om  # noqa: E402
from oracle import quant as oq  # noqa: E402
from oracle import route as orr  # noqa: E402

PATH = os.path.join(HERE, "golden.npz")

BLOCK = dict(H=512, F=512, E=8, k=2, g=128, bits=(1, 2, 3, 2, 3, 1, 2, 3), T=16, seed=2024)


def block_inputs(seed=BLOCK["seed"]):
    """Router weight, per-expert RTN triplets and activations of the block
    fixture, drawn in a fixed order from PCG64(seed).  Returns
    (gate fp16 [E, H], experts [{proj: (Q, s, z)}], x fp16 [T, H])."""
    rng = np.random.Generator(np.random.PCG64(seed))
    H, F, E, g = BLOCK["H"], BLOCK["F"], BLOCK["E"], BLOCK["g"]
    gate = (rng.standard_normal((E, H)) * 0.02).astype(np.float16)
    experts = []
    for e in range(E):
        b = BLOCK["bits"][e]
        ex = {}
        for name, (N, K) in (("gate_proj", (F, H)), ("up_proj", (F, H)), ("down_proj", (H, F))):
            W = (rng.standard_normal((N, K)) * 0.02).astype(np.float16)
            ex[name] = oq.rtn_quantize(W, b, g)
        experts.append(ex)
    x = rng.standard_normal((BLOCK["T"], H)).astype(np.float16)
    return gate, experts, x


def digest(gate, experts, x):
    h = hashlib.sha256()
    h.update(gate.tobytes())
    for ex in experts:
        for name in ("gate_proj", "up_proj", "down_proj"):
            for a in ex[name]:
                h.update(np.ascontiguousarray(a).tobytes())
    h.update(x.tobytes())
    return h.hexdigest()


def dense(triplet, N, K):
    Q, s, z = triplet
    return oq.dequant_hqq(Q, s, z).reshape(N, K).astype(np.float32)


def build():
    out = {}
    rng = np.random.Generator(np.random.PCG64(7))
    # RTN
    for b in (1, 2, 3, 4):
        W = (rng.standard_normal((8, 256)) * 0.02).astype(np.float16)
        W[3, 64:128] = np.float16(0.01)  # a constant group: the 1e-5 clamp path
        Q, s, z = oq.rtn_quantize(W, b, 64)
        out[f"rtn_b{b}_W"], out[f"rtn_b{b}_Q"], out[f"rtn_b{b}_s"], out[f"rtn_b{b}_z"] = W, Q, s, z
    # packing
    for b in (1, 2, 3, 4):
        codes = rng.integers(0, 1 << b, size=(16, 320)).astype(np.uint8)
        out[f"pack_b{b}_codes"] = codes
        out[f"pack_b{b}_words"] = oq.pack_cols(codes, b)
        out[f"pack_b{b}_build"] = oq.repack_build(codes[:, :256], b)
    # routing, fp16 gate
    x = rng.standard_normal((16, 512)).astype(np.float16)
    wg = (rng.standard_normal((8, 512)) * 0.02).astype(np.float16)
    lg = orr.router_logits(x.astype(np.float32), wg.astype(np.float32), "f16")
    out["route_x"], out["route_wg"], out["route_logits"] = x, wg, lg.astype(np.float16)
    for norm in (0, 1):
        idx, w = orr.topk_route(lg, 2, bool(norm))
        out[f"route_idx_n{norm}"], out[f"route_w_n{norm}"] = idx, w
    p = orr.permute(out["route_idx_n0"], 8)
    for key in ("counts", "offsets", "row_token", "row_pair", "inv_perm"):
        out[f"route_perm_{key}"] = p[key]
    # routing, fp32 gate, k = 6, shared experts
    wg32 = (rng.standard_normal((16, 512)) * 0.02).astype(np.float32)
    lg32 = orr.router_logits(x.astype(np.float32), wg32, "f32")
    idx32, w32 = orr.topk_route(lg32, 6, False)
    out["route32_wg"], out["route32_logits"], out["route32_idx"], out["route32_w"] = wg32, lg32, idx32, w32
    p = orr.permute(idx32, 16, n_shared=2)
    for key in ("counts", "offsets", "row_token", "row_pair", "inv_perm"):
        out[f"route32_perm_{key}"] = p[key]
    # one layer at the reference block-test shape
    gate, experts, xb = block_inputs()
    H, F = BLOCK["H"], BLOCK["F"]
    W1 = [dense(e["gate_proj"], F, H) for e in experts]
    W3 = [dense(e["up_proj"], F, H) for e in experts]
    W2 = [dense(e["down_proj"], H, F) for e in experts]
    y, lgb, idxb, wb = om.moe_forward(xb.astype(np.float32), gate.astype(np.float32), "f16", BLOCK["k"], False,
                                      W1, W3, W2)
    out["block_sha256"] = np.frombuffer(bytes.fromhex(digest(gate, experts, xb)), np.uint8)
    out["block_logits"], out["block_idx"], out["block_w"], out["block_out"] = lgb.astype(np.float16), idxb, wb, y
    return out


if __name__ == "__main__":
    data = build()
    np.savez_compressed(PATH, **data)
    print(f"wrote {PATH}: {len(data)} arrays, {os.path.getsize(PATH)} bytes")
