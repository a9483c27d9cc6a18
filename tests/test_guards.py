"""Load-time guards of the block mirror, on the CPU.

The truth tables are the reference's own known-answer cases:
tests/test_moe_block_equiv.py:255-314 (DeepSeek routing features and gate
semantics) and :316-331 (w1/w3 share bit-widths and strides).
"""

from types import SimpleNamespace

import pytest
import torch

from robustgemq_amd.moe_block import (check_deepseek_gate_matches, check_deepseek_routing_supported,
                                      check_w1_w3_aligned)


def _deepseek_config(**kw):
    base = dict(scoring_func="softmax", topk_method="greedy", norm_topk_prob=False, num_experts_per_tok=6,
                routed_scaling_factor=1.0)
    base.update(kw)
    return SimpleNamespace(**base)


class _Official:
    """A block loaded from the official modeling_deepseek.py via trust_remote_code
    lives in a transformers_modules.* package; only the module path matters."""


_Official.__module__ = "transformers_modules.deepseek.modeling_deepseek"


class _Builtin:
    """HF's built-in DeepseekV2 block."""


_Builtin.__module__ = "transformers.models.deepseek_v2.modeling_deepseek_v2"


def test_routing_guard_accepts_default():
    check_deepseek_routing_supported(_deepseek_config())
    cfg = _deepseek_config()
    del cfg.scoring_func  # the built-in config has no scoring_func: softmax
    check_deepseek_routing_supported(cfg)


@pytest.mark.parametrize("field,value", [("topk_method", "group_limited_greedy"), ("scoring_func", "sigmoid")])
def test_routing_guard_rejects_unsupported(field, value):
    with pytest.raises(AssertionError):
        check_deepseek_routing_supported(_deepseek_config(**{field: value}))


@pytest.mark.parametrize("official,norm,top_k,scaling,ok", [
    (True, False, 2, 1.0, True),
    (True, False, 2, 16.0, False),
    (True, True, 2, 16.0, True),
    (True, True, 1, 1.0, False),
    (False, False, 2, 1.0, True),
    (False, True, 2, 1.0, False),
    (False, False, 2, 16.0, False),
])
def test_deepseek_guard_truth_table(official, norm, top_k, scaling, ok):
    cfg = _deepseek_config(norm_topk_prob=norm, num_experts_per_tok=top_k, routed_scaling_factor=scaling)
    block = _Official() if official else _Builtin()
    if ok:
        check_deepseek_gate_matches(cfg, block)
    else:
        with pytest.raises(AssertionError):
            check_deepseek_gate_matches(cfg, block)


def test_w1_w3_alignment_guard():
    good = SimpleNamespace(w1_nbits=torch.tensor([2, 3]), w3_nbits=torch.tensor([2, 3]),
                           w1_wq_strides=torch.tensor([0, 128]), w3_wq_strides=torch.tensor([0, 128]))
    check_w1_w3_aligned(good)
    for field, value in (("w3_nbits", torch.tensor([2, 4])), ("w3_wq_strides", torch.tensor([0, 96]))):
        bad = SimpleNamespace(**vars(good))
        setattr(bad, field, value)
        with pytest.raises(AssertionError):
            check_w1_w3_aligned(bad)
