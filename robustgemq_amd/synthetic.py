"""Synthetic MoE layers shaped like the BASELINE configurations.

Weights are random (no checkpoints are available offline) and quantized with
the reference's RTN rule (gemq/quantizers/rtn.py:15-55), the way its own
synthetic tests build blocks (tests/test_moe_block_equiv.py:125-142,
tests/conftest.py:117-131).  Draw order from one CPU generator seeded with
`seed`: (1) per-expert bit assignment from randperm(E), (2) router weight
N(0, 0.02), (3) expert-major gate/up/down weights N(0, 0.02) cast to fp16,
(4) shared-expert weights.  Activations come from a second generator seeded
with seed + 1 so any token count can be drawn.
"""

import math
from dataclasses import dataclass, field

import torch

from .quantize import rtn_quantize


@dataclass(frozen=True)
class LayerConfig:
    name: str
    family: str            # olmoe | qwen3moe | mixtral | deepseekv2
    hidden: int
    inter: int
    n_experts: int
    top_k: int
    norm_topk: bool
    group_size: int
    bits: tuple            # ("fixed", b) | ("mix", {bits: count}) | ("list", (...))
    act_dtype: torch.dtype
    n_shared: int = 0
    shared_bits: int = 4
    zipf_s: float = 0.0    # > 0: add log p_e, p_e ~ rank^-s, to the router logits
    runs: dict = field(default_factory=dict, compare=False, hash=False)


CONFIGS = {
    # OLMoE-1B-7B shaped, uniform 2-bit, T = 128; and T = 2048, the
    # size BASELINE.json's north-star target quotes this layer at
    "olmoe_2bit": LayerConfig("olmoe_2bit", "olmoe", 2048, 1024, 64, 8, False, 64, ("fixed", 2),
                              torch.float16, runs={"prefill": (128, 2048)}),
    # mixed 2/3/4 bits 50/25/25
    "olmoe_mixed": LayerConfig("olmoe_mixed", "olmoe", 2048, 1024, 64, 8, False, 64,
                               ("mix", {2: 32, 3: 16, 4: 16}), torch.float16,
                               runs={"prefill": (512, 2048), "decode": (1, 8, 32)}),
    # Qwen3-30B-A3B shaped, average 2.5 bits (80 x 2, 32 x 3, 16 x 4)
    "qwen3_mixed": LayerConfig("qwen3_mixed", "qwen3moe", 2048, 768, 128, 8, True, 128,
                               ("mix", {2: 80, 3: 32, 4: 16}), torch.bfloat16,
                               runs={"prefill": (4096,), "decode": (1, 64)}),
    # DeepSeek-V2-Lite shaped, 2 shared experts (4-bit), Zipf routing
    "deepseek_v2_lite": LayerConfig("deepseek_v2_lite", "deepseekv2", 2048, 1408, 64, 6, False, 64,
                                    ("mix", {2: 32, 3: 32}), torch.float16, n_shared=2, shared_bits=4,
                                    zipf_s=1.1, runs={"prefill": (2048,)}),
    # Mixtral-8x7B shaped
    "mixtral_mixed": LayerConfig("mixtral_mixed", "mixtral", 4096, 14336, 8, 2, True, 64,
                                 ("mix", {2: 4, 3: 2, 4: 2}), torch.bfloat16,
                                 runs={"decode": (1, 16, 64), "prefill": (1024,)}),
    # Mixtral family at a test-sized shape (always-renormalised top-2, bf16)
    "mixtral_small": LayerConfig("mixtral_small", "mixtral", 1024, 3584, 8, 2, True, 64,
                                 ("mix", {2: 4, 3: 2, 4: 2}), torch.bfloat16, runs={"prefill": (300,)}),
    # the reference's own block-test shape (tests/test_moe_block_equiv.py:29-38)
    "ref_test": LayerConfig("ref_test", "olmoe", 512, 512, 8, 2, False, 128,
                            ("list", (1, 2, 3, 2, 3, 1, 2, 3)), torch.float16, runs={"prefill": (16,)}),
}


def expert_bits(cfg: LayerConfig, gen: torch.Generator):
    kind, spec = cfg.bits
    if kind == "fixed":
        torch.randperm(cfg.n_experts, generator=gen)  # keep the draw order uniform
        return [spec] * cfg.n_experts
    if kind == "list":
        torch.randperm(cfg.n_experts, generator=gen)
        assert len(spec) == cfg.n_experts
        return list(spec)
    perm = torch.randperm(cfg.n_experts, generator=gen).tolist()
    bits = [0] * cfg.n_experts
    pos = 0
    for b in sorted(spec):
        for e in perm[pos:pos + spec[b]]:
            bits[e] = b
        pos += spec[b]
    assert pos == cfg.n_experts
    return bits


def zipf_bias(cfg: LayerConfig, gen: torch.Generator):
    """log p_e with p_e proportional to rank_e^-s over a seeded permutation."""
    E = cfg.n_experts
    rank = torch.randperm(E, generator=gen).double() + 1.0
    p = rank.pow(-cfg.zipf_s)
    p = p / p.sum()
    return p.log().float()


def make_weights(cfg: LayerConfig, seed=0, quant_device="cpu", std=0.02):
    """Returns dict(bits, gate [E, H] fp16, experts [{gate_proj, up_proj,
    down_proj} -> QuantTriplet], shared dict | None, bias | None)."""
    gen = torch.Generator().manual_seed(seed)
    bits = expert_bits(cfg, gen)
    H, Fd, E = cfg.hidden, cfg.inter, cfg.n_experts
    gate = (torch.randn(E, H, generator=gen) * std).half()

    def q(shape, b):
        W = (torch.randn(*shape, generator=gen) * std).half().to(quant_device)
        return rtn_quantize(W, b, cfg.group_size)

    experts = []
    for e in range(E):
        experts.append({"gate_proj": q((Fd, H), bits[e]), "up_proj": q((Fd, H), bits[e]),
                        "down_proj": q((H, Fd), bits[e])})
    shared = None
    if cfg.n_shared:
        Fs = cfg.n_shared * Fd
        b = cfg.shared_bits
        shared = {"gate_proj": q((Fs, H), b), "up_proj": q((Fs, H), b), "down_proj": q((H, Fs), b)}
    bias = zipf_bias(cfg, gen) if cfg.zipf_s > 0 else None
    return dict(bits=bits, gate=gate, experts=experts, shared=shared, bias=bias)


def make_inputs(cfg: LayerConfig, T, seed=0, scale=1.0):
    gen = torch.Generator().manual_seed(seed + 1)
    return (torch.randn(T, cfg.hidden, generator=gen) * scale).to(cfg.act_dtype)


class _Cfg:
    """Minimal stand-in for the HF config fields the blocks read."""

    def __init__(self, **kw):
        self.__dict__.update(kw)


def hf_config(cfg: LayerConfig):
    common = dict(hidden_size=cfg.hidden, num_experts_per_tok=cfg.top_k, norm_topk_prob=cfg.norm_topk)
    if cfg.family == "olmoe":
        return _Cfg(intermediate_size=cfg.inter, num_experts=cfg.n_experts, **common)
    if cfg.family == "qwen3moe":
        return _Cfg(moe_intermediate_size=cfg.inter, num_experts=cfg.n_experts, **common)
    if cfg.family == "mixtral":
        return _Cfg(intermediate_size=cfg.inter, num_local_experts=cfg.n_experts, **common)
    if cfg.family == "deepseekv2":
        return _Cfg(moe_intermediate_size=cfg.inter, n_routed_experts=cfg.n_experts,
                    n_shared_experts=cfg.n_shared, topk_method="greedy", scoring_func="softmax",
                    routed_scaling_factor=1.0, **common)
    raise ValueError(cfg.family)


def build_block(cfg: LayerConfig, weights, device="cuda"):
    """A QuantFused*MoEBlock on `device` from make_weights() output."""
    from .moe_block import BLOCKS
    cls = BLOCKS[cfg.family]
    experts = [{k: t.to(device) for k, t in ex.items()} for ex in weights["experts"]]
    shared = None if weights["shared"] is None else {k: t.to(device) for k, t in weights["shared"].items()}
    block = cls.from_quantized(hf_config(cfg), weights["gate"].to(device), experts, shared=shared,
                               act_dtype=cfg.act_dtype)
    if weights["bias"] is not None:
        layer = block._layer
        from .ops import MoELayer
        block._layer = MoELayer(layer.gate_w, layer.w1, layer.w3, layer.w2, layer.top_k, layer.norm_topk,
                                layer.act_dtype, n_shared=layer.n_shared, logit_bias=weights["bias"].to(device),
                                one_token_act_softmax=layer.one_token_act_softmax)
    return block.to(device)


def flops(cfg: LayerConfig, T):
    """Algorithmic flops of one layer forward over T tokens:
    2*T*k*3*H*F + 2*T*H*E (+ 2*T*3*H*F_shared)."""
    f = 2 * T * cfg.top_k * 3 * cfg.hidden * cfg.inter + 2 * T * cfg.hidden * cfg.n_experts
    if cfg.n_shared:
        f += 2 * T * 3 * cfg.hidden * cfg.inter * cfg.n_shared
    return f


def expected_unique(cfg: LayerConfig, B):
    return cfg.n_experts * (1.0 - (1.0 - cfg.top_k / cfg.n_experts) ** B)
