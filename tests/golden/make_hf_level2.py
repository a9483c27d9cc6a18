"""Writes tests/golden/hf_level2.npz: outputs of the stock transformers MoE
blocks holding fake-quant weights, the comparator of the reference's Level-2
block test (tests/test_moe_block_equiv.py:197-235, :336-392), for
tests/test_gpu_hf_level2.py.

Same shapes as that test: hidden 512, expert intermediate 512, 8 experts,
top-2, group 128, per-expert bits [1, 2, 3, 2, 3, 1, 2, 3], DeepSeek with two
shared experts at 3 bits; 16 prompt tokens (x ~ N(0, 0.25)) and one decode
token.  Blocks are transformers' own (the installed 5.x classes, experts as
3-D gate_up_proj / down_proj parameters), built from CPU-seeded weights so
the GPU test rebuilds them bit for bit, with every expert slice replaced by
its RTN fake-quant weight (Q - z) * s (rtn.py:15-61, conftest.py:128-131) and
run in float32 on the CPU.  Also stored: the smallest gap between the k-th
and (k+1)-th router logit of any token, so the test can tell a routing
near-tie from a real difference.

Run from the repository root:  python tests/golden/make_hf_level2.py
"""

import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import quant as oq  # noqa: E402

H, F, E, K, G, T = 512, 512, 8, 2, 128, 16
BITS = [1, 2, 3, 2, 3, 1, 2, 3]
SHARED_BITS = 3
FAMILIES = ("olmoe", "qwen3moe", "mixtral", "deepseekv2")


def config(family):
    common = dict(hidden_size=H, num_experts_per_tok=K, num_hidden_layers=1, num_attention_heads=4,
                  num_key_value_heads=4, vocab_size=128)
    if family == "olmoe":
        from transformers.models.olmoe.configuration_olmoe import OlmoeConfig
        return OlmoeConfig(intermediate_size=F, num_experts=E, norm_topk_prob=False, **common)
    if family == "qwen3moe":
        from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig
        return Qwen3MoeConfig(intermediate_size=F, moe_intermediate_size=F, num_experts=E, norm_topk_prob=True,
                              **common)
    if family == "mixtral":
        from transformers.models.mixtral.configuration_mixtral import MixtralConfig
        return MixtralConfig(intermediate_size=F, num_local_experts=E, **common)
    from transformers.models.deepseek_v2.configuration_deepseek_v2 import DeepseekV2Config
    return DeepseekV2Config(intermediate_size=F, moe_intermediate_size=F, n_routed_experts=E, n_shared_experts=2,
                            first_k_dense_replace=0, **common)


def hf_block(family, cfg):
    """The stock block with deterministic weights N(0, 0.02) in fp16."""
    if family == "olmoe":
        from transformers.models.olmoe.modeling_olmoe import OlmoeSparseMoeBlock as cls
    elif family == "qwen3moe":
        from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeSparseMoeBlock as cls
    elif family == "mixtral":
        from transformers.models.mixtral.modeling_mixtral import MixtralSparseMoeBlock as cls
    else:
        from transformers.models.deepseek_v2.modeling_deepseek_v2 import DeepseekV2Moe as cls
    blk = cls(cfg).eval()
    gen = torch.Generator().manual_seed(FAMILIES.index(family) + 100)
    with torch.no_grad():
        for _, p in sorted(blk.named_parameters()):
            p.copy_((torch.randn(p.shape, generator=gen) * 0.02).half().to(p.dtype))
    return blk.half()


def inputs(family):
    gen = torch.Generator().manual_seed(FAMILIES.index(family) + 200)
    return (torch.randn(T + 1, H, generator=gen) * 0.5).half()


def fake_quant(W, nbits):
    """fp16 fake-quant weight of W [N, K] (rtn.py:15-61, conftest.py:128-131)."""
    N, Kd = W.shape
    Q, s, z = oq.rtn_quantize(W.numpy(), nbits, G)
    return torch.from_numpy(oq.dequant_hqq(Q, s, z).reshape(N, Kd))


def reference_block(family, blk):
    """A float32 copy of the block holding the fake-quant weights."""
    import copy
    ref = copy.deepcopy(blk)
    with torch.no_grad():
        ex = ref.experts
        for e in range(E):
            gu = ex.gate_up_proj.data[e]
            ex.gate_up_proj.data[e, :F] = fake_quant(gu[:F].clone(), BITS[e])
            ex.gate_up_proj.data[e, F:] = fake_quant(gu[F:].clone(), BITS[e])
            ex.down_proj.data[e] = fake_quant(ex.down_proj.data[e].clone(), BITS[e])
        sh = getattr(ref, "shared_experts", None)
        if sh is not None:
            for n in ("gate_proj", "up_proj", "down_proj"):
                lin = getattr(sh, n)
                lin.weight.data = fake_quant(lin.weight.data.clone(), SHARED_BITS)
    return ref.float()


def main():
    out = {}
    for family in FAMILIES:
        cfg = config(family)
        blk = hf_block(family, cfg)
        ref = reference_block(family, blk)
        x = inputs(family)
        with torch.no_grad():
            y_pre = ref(x[:T].float().reshape(1, T, H))
            y_dec = ref(x[T:].float().reshape(1, 1, H))
            lg = x.float() @ ref.gate.weight.data.float().T
        y_pre = y_pre[0] if isinstance(y_pre, tuple) else y_pre
        y_dec = y_dec[0] if isinstance(y_dec, tuple) else y_dec
        srt = torch.sort(lg, dim=1, descending=True).values
        gap = float((srt[:, K - 1] - srt[:, K]).min())
        out[f"{family}_x"] = x.numpy()
        out[f"{family}_prefill"] = y_pre.reshape(T, H).numpy().astype(np.float32)
        out[f"{family}_decode"] = y_dec.reshape(1, H).numpy().astype(np.float32)
        out[f"{family}_gap"] = np.float32(gap)
        print(f"{family}: |y| max {float(y_pre.abs().max()):.3e}, smallest top-{K} logit gap {gap:.3e}")
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "hf_level2.npz")
    np.savez_compressed(path, **out)
    print(path)


if __name__ == "__main__":
    main()
