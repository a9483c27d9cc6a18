"""Whole-model drop-in (robustgemq_amd/patch.py, the reference's
prepare_for_inference, gemq/inference/patch.py:165-181) on a two-layer
OLMoE-shaped toy model whose expert linears come from an HQQ checkpoint file
read without hqq: the installed blocks' outputs against the oracle on the
GemLite weights q * s + z' (fp32), at the expert path's bar."""

import numpy as np
import pytest
import torch

from conftest import relative_error, to_np
from oracle import moe as om

pytestmark = pytest.mark.gpu

MAX_ABS = 1e-2
REL_L2 = 1e-3


class _Expert(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.gate_proj = torch.nn.Identity()
        self.up_proj = torch.nn.Identity()
        self.down_proj = torch.nn.Identity()


class _MoE(torch.nn.Module):
    def __init__(self, H, E):
        super().__init__()
        self.gate = torch.nn.Linear(H, E, bias=False).half().cuda()
        self.experts = torch.nn.ModuleList([_Expert() for _ in range(E)])


class _Layer(torch.nn.Module):
    def __init__(self, H, E):
        super().__init__()
        self.mlp = _MoE(H, E)


class _Model(torch.nn.Module):
    def __init__(self, H, E, n_layers, config):
        super().__init__()
        self.model = torch.nn.Module()
        self.model.layers = torch.nn.ModuleList([_Layer(H, E) for _ in range(n_layers)])
        self.config = config


def test_prepare_for_inference_from_hqq_file(device, tmp_path):
    from robustgemq_amd import hqq_format as hf
    from robustgemq_amd.moe_block import QuantFusedOlmoeMoEBlock
    from robustgemq_amd.patch import prepare_for_inference
    from robustgemq_amd.quantize import rtn_quantize
    from robustgemq_amd.synthetic import _Cfg
    print("[patch] prepare_for_inference, 2 OLMoE-shaped layers from an HQQ file", flush=True)
    H, F, E, k, g, L = 256, 128, 6, 2, 64, 2
    bits = [1, 2, 3, 4, 2, 3]
    cfg = _Cfg(intermediate_size=F, num_experts=E, hidden_size=H, num_experts_per_tok=k, norm_topk_prob=False)
    model = _Model(H, E, L, cfg)
    gen = torch.Generator().manual_seed(3)
    states, dense = {}, {}
    for li in range(L):
        with torch.no_grad():
            model.model.layers[li].mlp.gate.weight.copy_((torch.randn(E, H, generator=gen) * 0.05).half())
        for e in range(E):
            for name, (N, K) in (("gate_proj", (F, H)), ("up_proj", (F, H)), ("down_proj", (H, F))):
                t = rtn_quantize((torch.randn(N, K, generator=gen) * 0.02).half(), bits[e], g)
                st = hf.HQQLinearState.from_quantized(t.Q, t.scales, t.zeros, t.shape, bits[e], g)
                key = f"model.layers.{li}.mlp.experts.{e}.{name}"
                states[key] = {"W_q": st.W_q, "meta": st.meta}
    path = tmp_path / "qmodel.pt"
    torch.save(states, path)
    prepare_for_inference(model, "allenai/OLMoE-1B-7B-0924", hqq_states=path)
    for li in range(L):
        blk = model.model.layers[li].mlp
        assert isinstance(blk, QuantFusedOlmoeMoEBlock)
        T = 9
        x = (torch.randn(T, H, generator=torch.Generator().manual_seed(li)) * 0.5).half()
        # the oracle on the GemLite weights the installed linears carry: q * s + z'
        W = {}
        for name in ("gate_proj", "up_proj", "down_proj"):
            W[name] = []
            for e in range(E):
                st = hf.HQQLinearState.from_state_dict(states[f"model.layers.{li}.mlp.experts.{e}.{name}"])
                q = hf.codes(st.W_q, st.meta).float()
                N, K = q.shape
                s = st.meta["scale"].float().reshape(N, K // g).half()
                zp = (-(st.meta["zero"].float().reshape(N, K // g) * s.float())).half()
                gi = torch.arange(K) // g
                W[name].append((q * s.float()[:, gi] + zp.float()[:, gi]).numpy())
        gate = blk._layer.gate_w.float().cpu().numpy()
        ref, _, _, _ = om.moe_forward(x.float().numpy(), gate, "f16", k, False, W["gate_proj"], W["up_proj"],
                                      W["down_proj"], ())
        out32, _ = blk._layer.forward(x.cuda(), out_dtype=torch.float32, want_logits=False)
        got = to_np(out32)
        err, mx = relative_error(got, ref), float(np.abs(got - ref).max())
        print(f"    layer {li}: rel-L2 {err:.3e} max-abs {mx:.3e}", flush=True)
        assert err <= REL_L2 and mx <= MAX_ABS
