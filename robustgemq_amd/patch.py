"""Drop-in installer for a whole HF model: HQQ linears become QuantLinear,
MoE blocks become QuantFused*MoEBlock (gemq/inference/patch.py:75-181).

    prepare_for_inference(model, "allenai/OLMoE-1B-7B-0924")

replaces, as the reference does, every HQQ linear of the model (any module
with W_q, meta and unpack(): hqq's HQQLinear, or hqq_format.HQQLinearState
in a module) and then each decoder layer's MoE block.  Checkpoint layers
already read into {name: HQQ layer state} (hqq_format.load_hqq_linears' input,
e.g. the file AutoHQQHFModel saves) are installed first when given, so a model
loads without the hqq package.
"""

import gc

import torch

from .hqq_format import load_hqq_linears
from .linear import QuantLinear
from .linear import replace_linear_recursive as _replace_children
from .moe_block import BLOCKS

# gemq/utils/model_utils.py:42-50 (the MoE models)
MODEL_FAMILY = {
    "mistralai/Mixtral-8x7B-v0.1": "mixtral",
    "deepseek-ai/DeepSeek-V2-Lite": "deepseekv2",
    "allenai/OLMoE-1B-7B-0924": "olmoe",
    "Qwen/Qwen3-30B-A3B": "qwen3moe",
}


def _is_hqq_linear(m):
    return hasattr(m, "W_q") and hasattr(m, "meta") and callable(getattr(m, "unpack", None))


def replace_linear_recursive(model, **kwargs):
    """Every HQQ linear below `model` -> QuantLinear.from_hqq_layer
    (patch.py:75-83)."""
    return _replace_children(model, lambda m: QuantLinear.from_hqq_layer(m, **kwargs) if _is_hqq_linear(m) else None)


def _family(model_name):
    if model_name in BLOCKS:
        return model_name
    if model_name not in MODEL_FAMILY:
        raise NotImplementedError(f"model {model_name!r} is not one of {sorted(MODEL_FAMILY)}")
    return MODEL_FAMILY[model_name]


def replace_moe_blocks(model, model_name, config):
    """Each decoder layer's HF MoE block -> QuantFused*MoEBlock.from_hf
    (patch.py:86-162): Mixtral's block_sparse_moe, the others' mlp; DeepSeek-V2
    skips its first (dense) layer; Qwen3-MoE replaces only the layers whose
    mlp is a sparse MoE block (mlp_only_layers / decoder_sparse_step)."""
    fam = _family(model_name)
    attr = "block_sparse_moe" if fam == "mixtral" else "mlp"
    for i, layer in enumerate(model.model.layers):
        if fam == "deepseekv2" and i == 0:
            continue
        org = getattr(layer, attr)
        if fam == "qwen3moe" and type(org).__name__ != "Qwen3MoeSparseMoeBlock":
            continue
        setattr(layer, attr, BLOCKS[fam].from_hf(config, org))
        del org
    gc.collect()
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    return model


def _set_module(root, dotted, value):
    parts = dotted.split(".")
    obj = root
    for p in parts[:-1]:
        obj = obj[int(p)] if p.isdigit() else getattr(obj, p)
    if parts[-1].isdigit():
        obj[int(parts[-1])] = value
    else:
        setattr(obj, parts[-1], value)


def install_hqq_states(model, states, device="cuda"):
    """Put QuantLinear built from HQQ layer states ({dotted module name: layer
    state}, or a file of them) at those names in the model."""
    for name, lin in load_hqq_linears(states, device=device).items():
        _set_module(model, name, lin)
    return model


def prepare_for_inference(model, model_name, hqq_states=None, device="cuda"):
    """patch.py:165-181 for the quantized model: (HQQ states installed if
    given), HQQ linears replaced, MoE blocks replaced."""
    if hqq_states is not None:
        install_hqq_states(model, hqq_states, device=device)
    replace_linear_recursive(model)
    replace_moe_blocks(model, model_name, model.config)
    gc.collect()
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    return model


__all__ = ["MODEL_FAMILY", "replace_linear_recursive", "replace_moe_blocks", "install_hqq_states",
           "prepare_for_inference"]
