"""Tiny random Hugging Face models, one per model type the SmoothQuant router accepts.

Shared by ``make_router_fixtures.py`` (which runs the reference router on them in the build
container) and ``tests/test_gpu_router.py`` (which runs this build's router on the same models on
the GPU box).  Only ``transformers`` is used here: nothing reads the reference tree.

Each model keeps the layer mix the router branches on: Qwen3.5 / Qwen3.5-MoE alternate
``linear_attention`` and ``full_attention`` layers; Qwen3-MoE has one dense layer
(``mlp_only_layers``) between packed-expert layers; the VL models carry a one-block vision tower
whose linears the router must leave alone.
"""
from __future__ import annotations

import torch

# model types in the order the fixtures list them; "mixtral" is outside the reference's
# allow-list (the reference raises ValueError for it)
MODEL_TYPES = ("llama", "qwen2", "qwen3", "qwen3_moe", "qwen2_5_vl", "qwen3_vl", "qwen3_5",
               "qwen3_5_moe", "qwen3_5_moe_text", "mixtral")

_TEXT = dict(hidden_size=64, intermediate_size=96, num_hidden_layers=4, num_attention_heads=4,
             num_key_value_heads=2, vocab_size=128, max_position_embeddings=64, bos_token_id=1, eos_token_id=2)
_VISION = dict(depth=1, hidden_size=32, intermediate_size=48, num_heads=2, out_hidden_size=64)
_LINEAR_ATTN = dict(linear_key_head_dim=16, linear_value_head_dim=16, linear_num_key_heads=2,
                    linear_num_value_heads=2, head_dim=16)
_LAYER_MIX = ["linear_attention", "full_attention", "linear_attention", "full_attention"]
_MOE = dict(num_experts=4, num_experts_per_tok=2, moe_intermediate_size=32)


def _config(model_type):
    from transformers import CONFIG_MAPPING
    cls = CONFIG_MAPPING[model_type]
    if model_type in ("llama", "qwen2", "qwen3", "mixtral"):
        kw = dict(_TEXT)
        if model_type == "mixtral":
            kw.update(num_local_experts=4, num_experts_per_tok=2)
        return cls(**kw)
    if model_type == "qwen3_moe":
        return cls(**_TEXT, num_experts=4, num_experts_per_tok=2, moe_intermediate_size=32, decoder_sparse_step=1,
                   mlp_only_layers=[1])
    if model_type in ("qwen2_5_vl", "qwen3_vl"):
        text = dict(_TEXT)
        if model_type == "qwen3_vl":
            text["head_dim"] = 16
        vision = dict(_VISION)
        if model_type == "qwen3_vl":
            vision["deepstack_visual_indexes"] = []
        return cls(text_config=text, vision_config=vision)
    if model_type == "qwen3_5":
        text = dict(_TEXT, **_LINEAR_ATTN, layer_types=_LAYER_MIX)
        return cls(text_config=text, vision_config=dict(_VISION))
    if model_type in ("qwen3_5_moe", "qwen3_5_moe_text"):
        text = dict(_TEXT, **_LINEAR_ATTN, **_MOE, layer_types=_LAYER_MIX, shared_expert_intermediate_size=48)
        text.pop("intermediate_size")
        if model_type == "qwen3_5_moe_text":
            return cls(**text)
        return cls(text_config=text, vision_config=dict(_VISION))
    raise ValueError(model_type)


def tiny_model(model_type, dtype=torch.float16, seed=0, layer_type_alias=True):
    """A randomly initialised model of ``model_type`` in ``dtype`` on the CPU, in eval mode.

    ``layer_type_alias``: Qwen3.5 decoder layers of the installed transformers (5.15) name their
    token mixer ``block_type``; the transformers the reference pins (5.6.0.dev0) named it
    ``layer_type``, which is the attribute the reference router reads.  With the alias each such
    layer also carries ``layer_type`` (same value), so the router sees the pinned version's
    layer."""
    from transformers import AutoModelForCausalLM, AutoModelForImageTextToText
    cfg = _config(model_type)
    torch.manual_seed(seed)
    if model_type in ("qwen2_5_vl", "qwen3_vl", "qwen3_5", "qwen3_5_moe"):
        model = AutoModelForImageTextToText.from_config(cfg, dtype=torch.float32)
    else:
        model = AutoModelForCausalLM.from_config(cfg, dtype=torch.float32)
    if layer_type_alias:
        for mod in model.modules():
            if hasattr(mod, "block_type") and not hasattr(mod, "layer_type"):
                mod.layer_type = mod.block_type
    return model.to(dtype).eval()


def module_kinds(model):
    """``{qualified name: class name}`` of every module whose class is a linear, a quantized
    linear or a packed-expert block: what the router swapped and what it left alone."""
    kinds = {}
    for name, mod in model.named_modules():
        cls = type(mod).__name__
        if cls in ("Linear", "SmoothQuantLinear", "SmoothQuantPackedMoeExperts") or cls.endswith("Experts"):
            kinds[name] = cls
    return kinds
