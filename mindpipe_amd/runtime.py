"""Runtime operator contract of the reference's deployed W8A8 path, on the gfx950 kernels.

``W8A8DynamicLinearMethod`` replaces ``AscendW8A8DynamicLinearMethod`` as patched by
MindPipe (``acceleration/runtime_patches/vllm_ascend.patch:3935-4033``): per-token
dynamic int8 quant (fp32 scale, the ``npu_dynamic_quant`` contract) then the int8
GEMM with the per-token x per-channel epilogue (``npu_quant_matmul``).
``fused_experts_w8a8`` replaces the MoE expert chain of ``_run_expert_tile``
(``vllm_ascend.patch:2356-2423``).  Layer attributes keep the reference's names
(``weight``, ``weight_scale``, ``weight_offset``, ``weight_scale_fp32``,
``_ascend_quant_config``); the weight stays ``[N, K]`` (the kernel reads that layout
directly, so no transpose or NZ cast is needed).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import ops

__all__ = ["W8A8DynamicLinearMethod", "fused_experts_w8a8", "dynamic_quant"]


def dynamic_quant(x: torch.Tensor):
    """``npu_dynamic_quant`` contract: ``(int8 [T,K], fp32 scale [T])`` with ``scale = absmax/127``."""
    return ops.quant_per_token_i8(x.contiguous(), False)


class W8A8DynamicLinearMethod:
    def __init__(self, transpose_weight: bool = False):
        # The reference transposes to [K, N] for the NPU format; the gfx950 kernel
        # consumes [N, K], so the default keeps the checkpoint layout.
        self.transpose_weight = transpose_weight

    def process_weights_after_loading(self, layer) -> None:
        """``vllm_ascend.patch:4022-4033``: flatten scale/offset, keep an fp32 scale copy."""
        w = layer.weight.data
        if self.transpose_weight:  # a [K, N] checkpoint is brought back to [N, K]
            w = w.transpose(0, 1)
        layer.weight.data = w.contiguous()
        layer.weight_scale.data = layer.weight_scale.data.flatten()
        layer.weight_scale_fp32 = layer.weight_scale.data.to(torch.float32).contiguous()
        if hasattr(layer, "weight_offset"):
            layer.weight_offset.data = layer.weight_offset.data.flatten()

    def apply(self, layer, x, bias: Optional[torch.Tensor] = None, tp_rank: Optional[int] = 0):
        """``vllm_ascend.patch:3935-4020``: ``x`` is a tensor (quantized here) or a pre-quantized
        ``(int8, scale)`` tuple; ``>2-D`` inputs are flattened and the output reshaped back;
        ``config['return_scale']`` returns ``(output, dynamic_scale)``."""
        config = getattr(layer, "_ascend_quant_config", {})
        output_shape = None
        if not isinstance(x, tuple):
            output_dtype = config.get("output_dtype", x.dtype)
            if x.dim() > 2:
                output_shape = x.shape[:-1]
                x = x.reshape(-1, x.shape[-1])
            quantized_x, dynamic_scale = dynamic_quant(x)
        else:
            output_dtype = config.get("output_dtype", getattr(layer, "params_dtype", torch.float16))
            quantized_x, dynamic_scale = x
            if quantized_x.dim() > 2:
                output_shape = quantized_x.shape[:-1]
                quantized_x = quantized_x.reshape(-1, quantized_x.shape[-1])
        if not config.get("pertoken_scale", True):
            raise NotImplementedError("the int8 GEMM epilogue needs the per-token scale")
        pertoken_scale = dynamic_scale.flatten().to(torch.float32).contiguous()
        output = ops.w8a8_gemm(quantized_x.contiguous(), pertoken_scale, layer.weight, layer.weight_scale_fp32,
                               bias, output_dtype)
        if output_shape is not None:
            output = output.reshape(*output_shape, output.shape[-1])
            dynamic_scale = dynamic_scale.reshape(*output_shape)
        return (output, dynamic_scale) if config.get("return_scale", False) else output


def fused_experts_w8a8(hidden_states: torch.Tensor, w1: torch.Tensor, w1_scale: torch.Tensor, w2: torch.Tensor,
                       w2_scale: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor,
                       output_dtype: Optional[torch.dtype] = None, **_unused) -> torch.Tensor:
    """W8A8 MoE experts: routing quant -> grouped GEMM1 + SwiGLU + requant -> grouped GEMM2
    -> weighted un-permute.  ``w1`` int8 ``[E, 2I, H]`` (gate rows first), ``w2`` int8
    ``[E, H, I]``, per-row scales ``[E, 2I]`` / ``[E, H]`` (any float dtype)."""
    return ops.moe_w8a8_forward(hidden_states.contiguous(), topk_ids, topk_weights, w1,
                                w1_scale.to(torch.float32).contiguous(), w2, w2_scale.to(torch.float32).contiguous(),
                                out_dtype=output_dtype or hidden_states.dtype)
