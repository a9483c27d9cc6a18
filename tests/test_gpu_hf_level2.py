"""The reference's Level-2 block check (tests/test_moe_block_equiv.py:197-235,
:336-392): a QuantFused*MoEBlock against the stock transformers block holding
the fake-quant weights, here for the installed transformers 5.x blocks, whose
experts are one module with 3-D gate_up_proj / down_proj parameters.

QuantFused*MoEBlock.from_hf(config, hf_block, bits, group_size, shared_bits)
quantizes those expert slices itself (RTN, rtn.py:15-55); the stock block's
outputs with the same fake-quant weights were written on the CPU by
tests/golden/make_hf_level2.py (float32, transformers' own forward), so no
stock block runs on the GPU.  Both dispatch branches are checked: 16 prompt
tokens (forward_n_tokens) and one decode token (forward_one_token), at the
layer bar of rel-L2 1e-3 (the reference allows 5e-2 for its own block).
"""

import os

import numpy as np
import pytest
import torch

from conftest import relative_error

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "hf_level2.npz")
REL_L2 = 1e-3


@pytest.mark.parametrize("family", ["olmoe", "qwen3moe", "mixtral", "deepseekv2"])
def test_fused_block_matches_stock_hf_block(device, family):
    pytest.importorskip("transformers")
    from golden import make_hf_level2 as mk

    from robustgemq_amd.moe_block import BLOCKS
    print(f"[hf level 2] {family}", flush=True)
    gold = np.load(GOLDEN)
    cfg = mk.config(family)
    hf = mk.hf_block(family, cfg).to(device)
    blk = BLOCKS[family].from_hf(cfg, hf, bits=mk.BITS, group_size=mk.G,
                                 shared_bits=mk.SHARED_BITS if family == "deepseekv2" else None)
    # the stacked reference attributes describe the per-expert bit-widths
    assert blk.w1_nbits.cpu().tolist() == mk.BITS and blk.block_group_size == mk.G
    x = torch.from_numpy(gold[f"{family}_x"]).to(device)
    assert torch.equal(x.cpu(), mk.inputs(family))  # same CPU-seeded inputs
    T, H = mk.T, mk.H
    pre = blk(x[:T].reshape(1, T, H))
    pre = pre[0] if isinstance(pre, tuple) else pre
    dec = blk(x[T:].reshape(1, 1, H))
    dec = dec[0] if isinstance(dec, tuple) else dec
    for name, got, want in (("prefill", pre.reshape(T, H), gold[f"{family}_prefill"]),
                            ("decode", dec.reshape(1, H), gold[f"{family}_decode"])):
        got = got.float().cpu().numpy()
        err = relative_error(got, want)
        print(f"    {name}: rel-L2 {err:.3e} (smallest top-k logit gap {float(gold[f'{family}_gap']):.2e})",
              flush=True)
        assert err <= REL_L2, (family, name, err)
