"""Quantization method adapters with the registry contract of the reference.

``BaseQuantizationMethod.apply_fake_quantization(model, tokenizer_bundle, args) -> dict``
(``algorithm/quantization/base.py:14-27``) is how MindPipe's workflow executor calls a method. The
two methods whose numerics this package implements are adapted here:

* ``SmoothQuantMethod`` (``ptq/smoothquant/method.py``). It checks the model type, bits and Q/K/V
  cache bits as the reference does, collects activation statistics (``get_act_scales``), smooths
  (``smooth_lm``) and swaps the linears for int8 ``SmoothQuantLinear`` / packed-expert modules
  (``quantize_model``). Its artifact dict has the reference's keys.
* ``AWQMethod`` (``ptq/awq/method.py:980-1182``). It runs the pseudo-quantization router
  ``pseudo_quantize_model_weight`` with ``{"zero_point": not weight_symmetric, "q_group_size":
  weight_group_size}``. The activation-aware scale / clip search (``run_awq``) is an offline
  calibration algorithm that this package does not implement: ``args.awq_search`` set raises.

Calibration data: the reference reads a named dataset through its own loader, which is not part of
this package. ``args.calibration_batches`` (an iterable of ``(token_ids, labels)``) supplies it here,
or ``args.smoothquant_act_scales_from`` names saved statistics (loaded with ``weights_only=True``).
"""
from __future__ import annotations

import logging
from abc import ABC, abstractmethod
from pathlib import Path
from typing import Any

import torch

from . import smoothquant as SQ
from . import w4a16 as W4

LOGGER = logging.getLogger(__name__)

__all__ = ["BaseQuantizationMethod", "SmoothQuantMethod", "AWQMethod", "METHODS"]


class BaseQuantizationMethod(ABC):
    """``base.py:14-27``: a method rewrites ``model`` in place and returns a JSON-able artifact dict."""

    name = "base"
    npu_ready: bool = False  # this package runs on the HIP device

    @abstractmethod
    def apply_fake_quantization(self, model, tokenizer_bundle, args) -> dict[str, Any]:
        raise NotImplementedError

    def resolve_output_dir(self, args) -> Path:
        slug = Path(str(args.model_path)).name or "model"
        spec = f"{self.name}_w{args.weight_bits}a{args.activation_bits}_seq{args.sequence_length}"
        out = Path(args.output_root) / slug / self.name / spec
        out.mkdir(parents=True, exist_ok=True)
        return out


def _alpha_tag(alpha: float) -> str:
    return f"{alpha:.2f}".rstrip("0").rstrip(".").replace(".", "p")


class SmoothQuantMethod(BaseQuantizationMethod):
    name = "smoothquant"
    default_calibration_dataset = "pileval"
    SUPPORTED_BIT_CONFIGS = {(8, 8)}

    def resolve_output_dir(self, args) -> Path:
        slug = Path(str(args.model_path)).name or "model"
        spec = (f"{self.name}_w{args.weight_bits}a{args.activation_bits}_seq{args.sequence_length}"
                f"_alpha{_alpha_tag(float(args.smoothquant_alpha))}")
        out = Path(args.output_root) / slug / self.name / spec
        out.mkdir(parents=True, exist_ok=True)
        return out

    def _validate_args(self, model, args) -> None:
        """The reference's checks (``method.py:85-108``): model type, W8A8 only, Q/K/V caches at 16 bits."""
        model_type = getattr(model.config, "model_type", None)
        if model_type not in SQ.SUPPORTED_MODEL_TYPES:
            raise NotImplementedError(
                "SmoothQuant currently supports LLaMA-, Qwen2/Qwen3/Qwen3.5/Qwen3.5-MoE-, and MiniCPM-style text "
                f"decoders only; got model_type={model_type!r}.")
        bits = (int(args.weight_bits), int(args.activation_bits))
        if bits not in self.SUPPORTED_BIT_CONFIGS:
            raise ValueError(f"SmoothQuant currently supports only W8A8; got W{bits[0]}A{bits[1]}.")
        if any(int(getattr(args, f, 16)) < 16 for f in ("query_bits", "key_bits", "value_bits")):
            raise ValueError("SmoothQuant fake-quant integration does not currently quantize Q/K/V caches; "
                             "keep --query_bits/--key_bits/--value_bits at 16.")

    def apply_fake_quantization(self, model, tokenizer_bundle, args) -> dict[str, Any]:
        self._validate_args(model, args)
        alpha = float(args.smoothquant_alpha)
        act_scales_path = None
        src = getattr(args, "smoothquant_act_scales_from", None)
        if src:
            act_scales_path = Path(src)
            act_scales = torch.load(act_scales_path, map_location="cpu", weights_only=True)
        else:
            batches = getattr(args, "calibration_batches", None)
            if batches is None:
                raise ValueError("SmoothQuantMethod needs args.calibration_batches ((token_ids, labels) pairs) or "
                                 "args.smoothquant_act_scales_from; the dataset loader is not part of this package")
            act_scales = SQ.get_act_scales(model, batches, getattr(args, "device", None))
            if getattr(args, "smoothquant_save_act_scales", False):
                act_scales_path = self.resolve_output_dir(args) / "act_scales.pt"
                torch.save(act_scales, act_scales_path)
        SQ.smooth_lm(model, act_scales, alpha=alpha)
        names = SQ.quantize_model(model, weight_bits=int(args.weight_bits), activation_bits=int(args.activation_bits),
                                  weight_quant="per_channel", act_quant="per_token", quantize_bmm_input=True)
        LOGGER.info("Replaced %s linear layers with SmoothQuant int8 modules (W%sA%s)", len(names),
                    args.weight_bits, args.activation_bits)
        out: dict[str, Any] = {
            "source_root": str(Path(__file__).resolve().parent),
            "smoothquant_config": {"alpha": alpha, "weight_bits": int(args.weight_bits),
                                   "activation_bits": int(args.activation_bits), "weight_quant": "per_channel",
                                   "activation_quant": "per_token", "quantize_bmm_input": True,
                                   "model_type": getattr(model.config, "model_type", None)},
            "quantized_linear_count": len(names),
            "quantized_linear_layers": {n: {"weight_bits": int(args.weight_bits),
                                            "activation_bits": int(args.activation_bits)} for n in names},
        }
        if act_scales_path is not None:
            out["act_scales_path"] = str(act_scales_path)
        return out


class AWQMethod(BaseQuantizationMethod):
    name = "awq"
    default_calibration_dataset = "pileval"

    def apply_fake_quantization(self, model, tokenizer_bundle, args) -> dict[str, Any]:
        if bool(getattr(args, "awq_search", False)):
            raise NotImplementedError("the AWQ scale / clip search (run_awq) is not part of this package; "
                                      "run with awq_search off to pseudo-quantize the weights")
        if int(args.activation_bits) < 16:
            LOGGER.warning("AWQ fake-quantizes weights only; activation_bits=%s adds no activation quantization.",
                           args.activation_bits)
        q_config = {"zero_point": not bool(args.weight_symmetric), "q_group_size": int(args.weight_group_size)}
        lin_attn = bool(getattr(args, "awq_qwen3_5_quantize_linear_attn", True))
        W4.pseudo_quantize_model_weight(model, w_bit=int(args.weight_bits), q_config=q_config,
                                        qwen3_5_quantize_linear_attn=lin_attn, device=getattr(args, "device", None))
        return {"source_root": str(Path(__file__).resolve().parent), "quantization_config": q_config,
                "awq_search_enabled": False, "awq_search_reused": False,
                "awq_qwen3_5_quantize_linear_attn": lin_attn,
                "resolved_weight_bits": {"visual": None, "connector": None, "llm": int(args.weight_bits)}}


METHODS = {"smoothquant": SmoothQuantMethod, "awq": AWQMethod}
