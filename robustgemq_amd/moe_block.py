"""QuantFused*MoEBlock: drop-in replacements for gemq/inference/moe_block.py.

Same class names, constructor (``from_hf(config, hf_block)``), attribute set
(w{1,2,3}_{wq,scales,zeros,nbits,group_sizes,wq_strides,zs_strides},
block_group_size, gate), dispatch (``forward`` -> ``forward_one_token`` when
B == S == 1, else ``forward_n_tokens``) and return convention
((hidden, router_logits | None) for Mixtral / OLMoE / Qwen3, a tensor for
DeepSeek) as the reference blocks (moe_block.py:140-309, :394-628, :688-858,
:918-1088).  Both forward branches run the same device-resident pipeline,
moeq_moe_forward: route -> permute -> grouped gate/up (SiLU*mul fused) ->
grouped down -> combine, one launch per stage, no host synchronisation, no
per-expert Python loop.

Two ways in:
  * ``from_hf(config, hf_block)`` -- experts already converted to GemLite-style
    linears (``W_q``, ``scales``, ``zeros`` = z' = -z*s, ``W_nbits``,
    ``group_size``) exactly as the reference requires (moe_block.py:720-722);
    weights are dequantized as q * s + z' like the reference kernels.
  * ``from_quantized(config, gate_weight, experts, shared=None)`` -- HQQ logical
    triplets (robustgemq_amd.quantize.QuantTriplet); weights are dequantized as
    (q - z) * s, bit-identical to the fake-quant weights.
"""

import torch
import torch.nn as nn

from . import _lib as L
from .experts import QuantProjection, pack_codes, unpack_words
from .ops import MoELayer


# ------------------------------------------------------------------- guards
def check_deepseek_routing_supported(config):
    """moe_block.py:18-28: softmax scoring and greedy top-k only."""
    scoring_func = getattr(config, "scoring_func", "softmax")
    assert scoring_func == "softmax", (
        f"fused block always uses softmax scoring, config asks for '{scoring_func}'")
    assert config.topk_method == "greedy", (
        f"fused block only implements topk_method='greedy', got '{config.topk_method}'")


def check_deepseek_gate_matches(config, hf_block):
    """moe_block.py:31-66: the fused block renormalizes iff norm_topk_prob and
    never applies routed_scaling_factor; accept only configs where the block
    being replaced combines weights the same way."""
    is_builtin = type(hf_block).__module__.startswith("transformers.models.deepseek_v2")
    normalizes = bool(config.norm_topk_prob)
    top_k = config.num_experts_per_tok
    if is_builtin:
        assert not normalizes, (
            "HF's built-in gate ignores norm_topk_prob while the fused block honours it; "
            "they agree only while it is False")
        assert config.routed_scaling_factor == 1.0, (
            f"built-in gate always scales by routed_scaling_factor "
            f"({config.routed_scaling_factor}), which the fused block never applies")
        return
    assert not (normalizes and top_k == 1), (
        "at top_k=1 the official gate scales, while the fused block would normalize the "
        "single weight to 1.0")
    if not (normalizes and top_k > 1):
        assert config.routed_scaling_factor == 1.0, (
            f"the official gate scales by routed_scaling_factor "
            f"({config.routed_scaling_factor}) whenever it does not normalize")


def check_w1_w3_aligned(fused_block):
    """moe_block.py:69-80: gate_proj and up_proj share bit-widths and strides."""
    assert torch.equal(fused_block.w1_nbits, fused_block.w3_nbits), (
        "w1 and w3 must share bit-widths: forward_one_token indexes w3 with w1's nbits")
    assert torch.equal(fused_block.w1_wq_strides, fused_block.w3_wq_strides), (
        "w1 and w3 must share packed strides: forward_one_token reads w3 at w1's offsets")


def _is_packed_linear(lin):
    return all(hasattr(lin, a) for a in ("W_q", "scales", "zeros", "W_nbits", "group_size"))


def _gemlite_part(lin):
    """(words [rows, N], scales [K/g, N], zeros [K/g, N], nbits) of a
    GemLite-style linear (the tensors from_hf concatenates, moe_block.py:725-733)."""
    return lin.W_q.data, lin.scales.data, lin.zeros.data, int(lin.W_nbits)


def _triplet_part(t):
    return pack_codes(t.codes(), t.nbits), t.scales_nk().half(), t.zeros_nk().half(), t.nbits


def _split_out(words, s, z, b, parts):
    """Split one projection along its output dim (N) into equal parts."""
    N = words.shape[1]
    w = N // parts
    return [(words[:, i * w:(i + 1) * w].contiguous(), s[:, i * w:(i + 1) * w].contiguous(),
             z[:, i * w:(i + 1) * w].contiguous(), b) for i in range(parts)]


def _split_in(words, s, z, b, K, group_size, parts):
    """Split one projection along its input dim (K) into equal parts."""
    codes = unpack_words(words, b, K)  # [N, K]
    kw = K // parts
    gw = kw // group_size
    out = []
    for i in range(parts):
        c = codes[:, i * kw:(i + 1) * kw].contiguous()
        out.append((pack_codes(c, b), s[i * gw:(i + 1) * gw].contiguous(), z[i * gw:(i + 1) * gw].contiguous(), b))
    return out


def _projection(parts, K, N, group_size, dq_mode):
    return QuantProjection([p[0] for p in parts], [p[1] for p in parts], [p[2] for p in parts],
                           [p[3] for p in parts], K, N, group_size, dq_mode)


class _QuantFusedMoEBase(nn.Module):
    """Shared implementation; subclasses fix config field names and routing."""

    _proj_names = ("gate_proj", "up_proj", "down_proj")  # -> w1, w3, w2
    _always_renorm = False
    _one_token_act_softmax = False  # Mixtral: 16-bit softmax in forward_one_token
    _gate_fp32 = False
    _returns_logits = True
    _family = "?"

    def __init__(self, config):
        super().__init__()
        self._init_dims(config)
        self.gate = nn.Linear(self.hidden_dim, self.num_experts, bias=False)
        for p in ("w1", "w2", "w3"):
            for a in ("wq", "scales", "zeros", "nbits", "group_sizes", "wq_strides", "zs_strides"):
                setattr(self, f"{p}_{a}", None)
        self.block_group_size = None
        self.num_shared_experts = getattr(self, "num_shared_experts", 0)
        self._layer = None

    # -- construction -----------------------------------------------------
    def _install(self, w1, w3, w2, gate_weight, act_dtype, shared=None):
        for name, proj in (("w1", w1), ("w3", w3), ("w2", w2)):
            E = self.num_experts
            # reference attributes describe the routed experts only
            for a in ("nbits", "group_sizes", "wq_strides", "zs_strides"):
                setattr(self, f"{name}_{a}", getattr(proj, a)[:E])
            setattr(self, f"{name}_wq", proj.wq)
            setattr(self, f"{name}_scales", proj.scales)
            setattr(self, f"{name}_zeros", proj.zeros)
        gs = {w1.group_size, w3.group_size, w2.group_size}
        assert len(gs) == 1, "Group sizes must be the same across all experts."
        self.block_group_size = gs.pop()
        self.gate.weight.data = gate_weight.detach().clone()
        check_w1_w3_aligned(self)
        gate_w = self.gate.weight.data.float() if self._gate_fp32 else self.gate.weight.data.to(act_dtype)
        n_shared = shared if shared else 0
        self._layer = MoELayer(gate_w, w1, w3, w2, self.top_k, self._renorm(), act_dtype, n_shared=n_shared,
                               one_token_act_softmax=self._one_token_act_softmax)
        return self

    def _renorm(self):
        return True if self._always_renorm else bool(self.norm_topk_prob)

    @classmethod
    def from_hf(cls, config, hf_block, bits=None, group_size=None, shared_bits=None):
        """Build the block from an HF MoE block (patch.py:86-162 calls this
        for every MoE layer).  Two layouts:

        * experts as a list of per-expert modules whose linears are already
          GemLite-converted (transformers 4.x, the reference's from_hf,
          moe_block.py:715-761 and family variants): their packed words are
          stacked and dequantize as q * s + z', like the reference kernels;
        * experts as one module with 3-D parameters (transformers 5.x:
          experts.gate_up_proj [E, 2F, H], experts.down_proj [E, H, F], and
          DeepSeek's shared_experts MLP): every expert slice is quantized here
          with the RTN rule (gemq/quantizers/rtn.py:15-55) at `bits` (one
          int, or one per expert), `group_size` and `shared_bits`, and the
          block computes with the fake-quant weights (q - z) * s, as
          from_quantized does."""
        if hasattr(hf_block.experts, "gate_up_proj"):
            return cls._from_fused_experts(config, hf_block, bits, group_size, shared_bits)
        block = cls(config)
        experts = cls._hf_experts(hf_block)
        n1, n3, n2 = cls._proj_names
        if not _is_packed_linear(getattr(experts[0], n1)):
            raise ValueError(f"Expected linears in {cls._family} block. Please patch and replace them first.")
        parts = {n: [_gemlite_part(getattr(ex, n)) for ex in experts] for n in (n1, n3, n2)}
        g = int(getattr(experts[0], n1).group_size)
        H, Fd = block.hidden_dim, block.ffn_dim
        shared = block._hf_shared_parts(config, hf_block, g)
        n_sh = 0
        if shared is not None:
            n_sh = len(shared[0])
            for i, n in enumerate((n1, n3, n2)):
                parts[n] = parts[n] + shared[i]
        w1 = _projection(parts[n1], H, Fd, g, L.DQ_AFFINE)
        w3 = _projection(parts[n3], H, Fd, g, L.DQ_AFFINE)
        w2 = _projection(parts[n2], Fd, H, g, L.DQ_AFFINE)
        act = hf_block.gate.weight.dtype if hf_block.gate.weight.dtype != torch.float32 else torch.float16
        return block._install(w1, w3, w2, hf_block.gate.weight.data, act, shared=n_sh)

    @classmethod
    def _from_fused_experts(cls, config, hf_block, bits, group_size, shared_bits):
        """transformers 5.x layout: gate_up_proj[e] holds gate_proj (rows
        0..F-1) over up_proj (rows F..2F-1), as OlmoeExperts.forward splits
        it with .chunk(2)."""
        from .quantize import rtn_quantize
        ex = hf_block.experts
        E, F2, H = ex.gate_up_proj.shape
        F = F2 // 2
        if bits is None or group_size is None:
            raise ValueError("a block with fused 3-D expert weights is quantized here: pass bits and group_size")
        bl = [int(bits)] * E if isinstance(bits, int) else [int(b) for b in bits]
        if len(bl) != E:
            raise ValueError(f"bits lists {len(bl)} experts, the block has {E}")
        g = int(group_size)
        gu_all, dn_all = ex.gate_up_proj.data, ex.down_proj.data
        experts = []
        for e in range(E):
            gu = gu_all[e].to(torch.float16)
            experts.append({"gate_proj": rtn_quantize(gu[:F].contiguous(), bl[e], g),
                            "up_proj": rtn_quantize(gu[F:].contiguous(), bl[e], g),
                            "down_proj": rtn_quantize(dn_all[e].to(torch.float16).contiguous(), bl[e], g)})
        shared = None
        sh = getattr(hf_block, "shared_experts", None)
        if sh is not None:
            if shared_bits is None:
                raise ValueError("the block has shared experts: pass shared_bits")
            shared = {n: rtn_quantize(getattr(sh, n).weight.data.to(torch.float16).contiguous(), int(shared_bits), g)
                      for n in ("gate_proj", "up_proj", "down_proj")}
        gw = hf_block.gate.weight.data
        act = gw.dtype if gw.dtype != torch.float32 else torch.float16
        return cls.from_quantized(config, gw, experts, shared=shared, act_dtype=act)

    @classmethod
    def from_quantized(cls, config, gate_weight, experts, shared=None, act_dtype=torch.float16):
        """From HQQ logical triplets: ``experts`` is a list (one per routed
        expert) of dicts {"gate_proj", "up_proj", "down_proj"} -> QuantTriplet;
        ``shared`` (DeepSeek) the same dict for the fused shared MLP
        ([n_shared * F, H] gate/up, [H, n_shared * F] down).  Weights
        dequantize as (q - z) * s, the fake-quant weights bit for bit."""
        block = cls(config)
        H, Fd = block.hidden_dim, block.ffn_dim
        g = experts[0]["gate_proj"].group_size
        parts = {n: [_triplet_part(ex[n]) for ex in experts] for n in ("gate_proj", "up_proj", "down_proj")}
        n_sh = 0
        if shared is not None:
            n_sh = shared["gate_proj"].shape[0] // Fd
            gp, up, dp = (_triplet_part(shared[n]) for n in ("gate_proj", "up_proj", "down_proj"))
            parts["gate_proj"] += _split_out(*gp, n_sh)
            parts["up_proj"] += _split_out(*up, n_sh)
            parts["down_proj"] += _split_in(*dp, n_sh * Fd, g, n_sh)
        w1 = _projection(parts["gate_proj"], H, Fd, g, L.DQ_HQQ)
        w3 = _projection(parts["up_proj"], H, Fd, g, L.DQ_HQQ)
        w2 = _projection(parts["down_proj"], Fd, H, g, L.DQ_HQQ)
        return block._install(w1, w3, w2, gate_weight, act_dtype, shared=n_sh)

    @staticmethod
    def _hf_experts(hf_block):
        return list(hf_block.experts)

    def _hf_shared_parts(self, config, hf_block, g):
        return None

    # -- forward ----------------------------------------------------------
    def _run(self, hidden_states, want_logits, one_token=False):
        if self._layer is None:
            raise RuntimeError("block has no weights: build it with from_hf() or from_quantized()")
        B, S, H = hidden_states.shape
        x = hidden_states.reshape(-1, H)
        out, logits = self._layer.forward(x, want_logits=want_logits, one_token=one_token)
        return out.reshape(B, S, H), logits

    def forward_n_tokens(self, hidden_states):
        """Any number of tokens in one device-resident pass (replaces the
        per-expert loop of moe_block.py:781-815)."""
        out, logits = self._run(hidden_states, want_logits=self._returns_logits)
        return (out, logits) if self._returns_logits else out

    def forward_one_token(self, hidden_states):
        """Single-token decode (moe_block.py:817-853); capture-safe."""
        B, S, H = hidden_states.shape
        assert B * S == 1, f"This function only supports single token forward. But got {B * S} tokens."
        out, _ = self._run(hidden_states, want_logits=False, one_token=True)
        return (out, None) if self._returns_logits else out

    def forward(self, hidden_states):
        if hidden_states.shape[0] == hidden_states.shape[1] == 1:
            return self.forward_one_token(hidden_states)
        return self.forward_n_tokens(hidden_states)


class QuantFusedOlmoeMoEBlock(_QuantFusedMoEBase):
    """gemq/inference/moe_block.py:688-858."""
    _family = "OlmoeSparseMoeBlock"

    def _init_dims(self, config):
        self.hidden_dim = config.hidden_size
        self.ffn_dim = config.intermediate_size
        self.num_experts = config.num_experts
        self.top_k = config.num_experts_per_tok
        self.norm_topk_prob = config.norm_topk_prob


class QuantFusedQwen3MoeMoEBlock(_QuantFusedMoEBase):
    """gemq/inference/moe_block.py:918-1088."""
    _family = "Qwen3MoeSparseMoeBlock"

    def _init_dims(self, config):
        self.hidden_dim = config.hidden_size
        self.ffn_dim = config.moe_intermediate_size
        self.num_experts = config.num_experts
        self.top_k = config.num_experts_per_tok
        self.norm_topk_prob = config.norm_topk_prob


class QuantFusedMixtralMoEBlock(_QuantFusedMoEBase):
    """gemq/inference/moe_block.py:140-309 (routing always renormalized)."""
    _family = "MixtralSparseMoeBlock"
    _proj_names = ("w1", "w3", "w2")
    _always_renorm = True
    # forward_one_token ranks and renormalises softmax probabilities in the
    # activation dtype (moe_block.py:280-283), forward_n_tokens in fp32 (:245-249)
    _one_token_act_softmax = True

    def _init_dims(self, config):
        self.hidden_dim = config.hidden_size
        self.ffn_dim = config.intermediate_size
        self.num_experts = config.num_local_experts
        self.top_k = config.num_experts_per_tok
        self.norm_topk_prob = True

    @classmethod
    def from_quantized(cls, config, gate_weight, experts, shared=None, act_dtype=torch.float16):
        ren = [{"gate_proj": e.get("w1", e.get("gate_proj")), "up_proj": e.get("w3", e.get("up_proj")),
                "down_proj": e.get("w2", e.get("down_proj"))} for e in experts]
        return super().from_quantized(config, gate_weight, ren, shared=None, act_dtype=act_dtype)


class QuantFusedDeepseekV2MoEBlock(_QuantFusedMoEBase):
    """gemq/inference/moe_block.py:394-628: fp32 gate, shared experts added
    unweighted; returns a tensor."""
    _family = "DeepseekV2MoE"
    _gate_fp32 = True
    _returns_logits = False

    def __init__(self, config):
        check_deepseek_routing_supported(config)
        self.num_shared_experts = config.n_shared_experts
        super().__init__(config)
        self.shared_nbits, self.shared_group_size = None, None

    def _init_dims(self, config):
        self.hidden_dim = config.hidden_size
        self.ffn_dim = config.moe_intermediate_size
        self.num_experts = config.n_routed_experts
        self.top_k = config.num_experts_per_tok
        self.norm_topk_prob = config.norm_topk_prob

    @classmethod
    def from_hf(cls, config, hf_block, bits=None, group_size=None, shared_bits=None):
        check_deepseek_gate_matches(config, hf_block)
        return super().from_hf(config, hf_block, bits=bits, group_size=group_size, shared_bits=shared_bits)

    def _hf_shared_parts(self, config, hf_block, g):
        sh = hf_block.shared_experts
        n_sh = int(config.n_shared_experts)
        gp, up, dp = (_gemlite_part(getattr(sh, n)) for n in ("gate_proj", "up_proj", "down_proj"))
        bits = {gp[3], up[3], dp[3]}
        assert len(bits) == 1, "the shared-expert kernels assume one bit-width (moe_block.py:487-504)"
        self.shared_nbits, self.shared_group_size = gp[3], g
        return (_split_out(*gp, n_sh), _split_out(*up, n_sh), _split_in(*dp, n_sh * self.ffn_dim, g, n_sh))

    @classmethod
    def from_quantized(cls, config, gate_weight, experts, shared=None, act_dtype=torch.float16):
        block = super().from_quantized(config, gate_weight, experts, shared=shared, act_dtype=act_dtype)
        if shared is not None:
            block.shared_nbits = shared["gate_proj"].nbits
            block.shared_group_size = shared["gate_proj"].group_size
        return block


BLOCKS = {
    "olmoe": QuantFusedOlmoeMoEBlock,
    "qwen3moe": QuantFusedQwen3MoeMoEBlock,
    "mixtral": QuantFusedMixtralMoEBlock,
    "deepseekv2": QuantFusedDeepseekV2MoEBlock,
}
