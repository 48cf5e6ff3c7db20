"""SmoothQuant W8A8 modules with the reference's API, backed by the gfx950 kernels.

Mirrors ``algorithm/quantization/ptq/smoothquant/source/smoothquant/fake_quant.py``
(``quantize_weight_per_channel_absmax`` :10-19, ``quantize_activation_per_token_absmax``
:22-31, ``SmoothQuantLinear`` :38-121, ``SmoothQuantPackedMoeExperts`` :124-198,
``quantize_llama_like`` / ``quantize_model`` :201-457) and the smoothing helpers of
``smooth.py:7-25,91-101``.  Same constructor arguments, attribute names and
``forward`` signatures; the difference is that the weights are held as real int8
codes with per-row scales and ``forward`` runs the per-token int8 quantizer and the
int8 MFMA GEMM (or the MoE chain) instead of fake-quant ``F.linear``.

Widths: ``weight_bits`` / ``activation_bits`` of 8 run the int8 path above; 2..7 keep int8
codes of the narrower rule (``q_max = 2^(n-1) - 1``) and >= 16 leave the operand unquantized, as
the reference does; those combinations multiply on the dequantising GEMM, which rounds each
operand element as the reference's fake-quant tensors are.  9..15 bits would need codes wider
than int8 and raise ``NotImplementedError``.

Scale rule (``scale_rule``):
  * ``"fake"`` (default for the modules): the arithmetic of the reference's
    ``quantize_*_absmax`` in the module dtype (fp16 or bf16) -- ``q * s`` is the value the
    reference's fake quantizer rounds to, and outputs match its ``F.linear`` on the
    fake-quant tensors to the output rounding.  The packed MoE experts additionally round
    gate, up, ``silu(gate)``, ``h``, the down output, the router-weighted rows and every
    ``index_add_`` step as the reference forward does.
  * ``"export"``: the fp32 rule of the Ascend W8A8 export / runtime
    (``npu_dynamic_quant`` contract), the one ``runtime.W8A8DynamicLinearMethod`` uses.
"""
from __future__ import annotations

from functools import partial
from typing import List, Optional

import torch
import torch.nn.functional as F
from torch import nn

from . import ops

__all__ = [
    "quantize_weight_per_channel_absmax",
    "quantize_activation_per_token_absmax",
    "SmoothQuantLinear",
    "SmoothQuantPackedMoeExperts",
    "quantize_llama_like",
    "quantize_model",
    "text_backbone",
    "SUPPORTED_MODEL_TYPES",
    "compute_smooth_scales",
    "smooth_ln_fcs_llama_like",
    "smooth_ln_fcs_qwen3_5",
    "smooth_qwen3_moe_ffn",
    "smooth_qwen3_5_moe_ffn",
    "smooth_lm",
    "get_act_scales",
]


def _require_gpu(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{what}: mindpipe_amd runs on the GPU only (tensor is on {t.device})")


_FAKE_DTYPES = (torch.float16, torch.bfloat16)


def _width(bits, what: str) -> int:
    """The code width of a quantizer argument: 2..8, or >= 16 for no quantization."""
    b = int(bits)
    if b >= 16 or 2 <= b <= 8:
        return b
    raise NotImplementedError(f"{what}={b}: this build quantizes to 2..8-bit int8 codes (or >= 16: none)")


def _row_codes(t2: torch.Tensor, n_bits: int):
    """Fake-rule codes of the rows of a 2-D fp16 / bf16 tensor at ``n_bits`` (2..8): ``(int8 q,
    fp32 s)`` with ``r(q * s)`` the reference's fake-quant value."""
    if n_bits == 8:
        q, s = ops.quant_per_token_i8(t2, True)
        return q, s.float()
    return ops.fake_quant_rows(t2, n_bits)


@torch.no_grad()
def quantize_weight_per_channel_absmax(weight: torch.Tensor, n_bits: int = 8) -> torch.Tensor:
    """Fake-quantized weight (``q * s`` in the weight dtype), as ``fake_quant.py:10-19`` returns it.

    The codes come from the GPU quantizer (fake rule in the weight's dtype, fp16 or bf16);
    the returned tensor holds the same values as the reference's (the sign of an exact zero
    is not carried by int8 codes).  ``n_bits >= 16`` returns a copy, like the reference.
    """
    n_bits = _width(n_bits, "n_bits")
    if n_bits >= 16:
        return weight.detach().clone()
    _require_gpu(weight, "quantize_weight_per_channel_absmax")
    shape = weight.shape
    w2 = weight.detach().reshape(-1, shape[-1]).contiguous()
    if w2.dtype not in _FAKE_DTYPES:
        raise NotImplementedError("the fake-quant rule takes fp16 or bf16 weights")
    if n_bits == 8:
        q, s32, _ = ops.w8_quantize_per_channel(w2, "fake")
    else:
        q, s32 = ops.fake_quant_rows(w2, n_bits)
    return (q.float() * s32[:, None]).to(weight.dtype).reshape(shape)


@torch.no_grad()
def quantize_activation_per_token_absmax(tensor: torch.Tensor, n_bits: int = 8) -> torch.Tensor:
    """Fake-quantized activation (``q * s`` in the input dtype), as ``fake_quant.py:22-31`` returns it."""
    n_bits = _width(n_bits, "n_bits")
    if n_bits >= 16:
        return tensor
    _require_gpu(tensor, "quantize_activation_per_token_absmax")
    if tensor.dtype not in _FAKE_DTYPES:
        raise NotImplementedError("the fake-quant rule takes fp16 or bf16 activations")
    q, s = _row_codes(tensor.contiguous(), n_bits)
    return (q.float() * s.unsqueeze(-1)).to(tensor.dtype)


class SmoothQuantLinear(nn.Module):
    """W8A8 linear: int8 ``weight [N,K]`` + fp32 ``weight_scale [N]``, per-token int8 activations.

    Constructor and ``from_float`` follow ``fake_quant.py:38-113``.  ``forward`` =
    per-token int8 quant of ``x`` -> int8 MFMA GEMM with the ``(acc * s_tok) * s_ch
    (+ bias)`` epilogue -> optional output fake-quant (``quantize_output``, :77-82).
    """

    def __init__(self, in_features, out_features, bias=True, weight_bits=8, activation_bits=8,
                 act_quant="per_token", quantize_output=False, dtype=torch.float16, scale_rule="fake"):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.weight_bits = _width(weight_bits, "weight_bits")
        self.activation_bits = _width(activation_bits, "activation_bits")
        if act_quant != "per_token":
            raise ValueError(f"Invalid act_quant: {act_quant}")
        if scale_rule not in ("fake", "export"):
            raise ValueError(f"Invalid scale_rule: {scale_rule}")
        if scale_rule == "export" and (self.weight_bits, self.activation_bits) != (8, 8):
            raise ValueError("scale_rule='export' is the W8A8 runtime rule (8-bit weights and activations)")
        self.scale_rule = scale_rule
        self.dtype = dtype
        wdt = torch.int8 if self.weight_bits < 16 else dtype
        self.register_buffer("weight", torch.zeros((out_features, in_features), dtype=wdt, requires_grad=False))
        self.register_buffer("weight_scale", torch.ones((out_features,), dtype=torch.float32))
        if bias:
            self.register_buffer("bias", torch.zeros((out_features,), dtype=dtype, requires_grad=False))
        else:
            self.register_buffer("bias", None)
        self.weight_quant_name = "per_channel" if self.weight_bits < 16 else "none"
        self.act_quant_name = act_quant if self.activation_bits < 16 else "none"
        self.output_quant_name = self.act_quant_name if quantize_output else "none"
        self.act_quant = (partial(quantize_activation_per_token_absmax, n_bits=self.activation_bits)
                          if self.activation_bits < 16 else (lambda t: t))

    @property
    def quantize_output(self) -> bool:
        return self.output_quant_name != "none"

    def output_quant(self, y):
        if self.output_quant_name == "none":
            return y
        return quantize_activation_per_token_absmax(y, self.activation_bits)

    def dequantized_weight(self) -> torch.Tensor:
        """The fake-quant weight the reference module would hold (``q * s``)."""
        if self.weight_bits >= 16:
            return self.weight
        return (self.weight.float() * self.weight_scale[:, None]).to(self.dtype)

    @property
    def _w8a8(self) -> bool:
        return self.weight_bits == 8 and self.activation_bits == 8

    def _linear_any_width(self, x):
        """``F.linear(act_quant(x), weight, bias)`` at widths other than W8A8 on the dequantising
        GEMM: each operand int8 codes of its width (rounded as ``r(q * s)``) or plain values."""
        if x.dtype not in _FAKE_DTYPES:
            raise NotImplementedError("the fake-quant linear runs in fp16 or bf16")
        x2 = x.reshape(-1, self.in_features).contiguous()
        if self.activation_bits < 16:
            qa, sa = _row_codes(x2, self.activation_bits)
        else:
            qa, sa = x2, None
        if self.weight_bits < 16:
            qb, sb = self.weight, self.weight_scale
        else:
            if self.weight.dtype != x.dtype:
                raise RuntimeError(f"input dtype {x.dtype} does not match the weight's {self.weight.dtype}")
            qb, sb = self.weight, None
        bias = None if self.bias is None else self.bias.to(x.dtype)
        y = ops.dq_linear(qa, sa, qb, sb, bias, x.dtype)
        return y.reshape(*x.shape[:-1], self.out_features)

    @torch.no_grad()
    def forward(self, x):
        _require_gpu(x, "SmoothQuantLinear")
        if not self._w8a8:
            return self.output_quant(self._linear_any_width(x))
        fake, q, s = self._input_codes(x)
        if self._fused_output_quant(x, fake):
            qo, so = self._output_codes(q, s, x.dtype)
            return (qo.float() * so.unsqueeze(-1)).to(x.dtype)
        return self.output_quant(self._linear(x, fake, q, s))

    def _input_codes(self, x):
        fake = self.scale_rule == "fake"
        if fake and x.dtype not in _FAKE_DTYPES:
            raise NotImplementedError("the fake scale rule takes fp16 or bf16 activations")
        q, s = ops.quant_per_token_i8(x.contiguous(), fake)
        return fake, q, s

    def _linear(self, x, fake, q, s):
        """The linear's output before any output quant."""
        if fake and x.dtype == torch.bfloat16:
            # bf16 keeps 8 significant bits: the reference multiplies the bf16-rounded fake values
            # r(q * s), which the int8 product of q * s misses by ~3e-3; the dequantising GEMM
            # rounds each element as the reference does
            bias = None if self.bias is None else self.bias.to(torch.bfloat16)
            return ops.w8a8_gemm_fake(q, s.float().contiguous(), self.weight, self.weight_scale, bias, x.dtype)
        return ops.w8a8_gemm(q, s.float().contiguous(), self.weight, self.weight_scale, self.bias, x.dtype)

    def _fused_output_quant(self, x, fake: bool) -> bool:
        """The output quant runs in the GEMM epilogue (``w8a8_gemm_quant_out``) for 8-bit outputs of
        the int8 GEMM (not the bf16 fake-rule linear, which rounds its operands) when K % 128 == 0."""
        return (self.output_quant_name != "none" and self.activation_bits == 8 and self.in_features % 128 == 0
                and not (fake and x.dtype == torch.bfloat16))

    def _output_codes(self, q, s, dtype):
        lead = q.shape[:-1]
        bias = None if self.bias is None else self.bias.to(dtype)
        _, qo, so = ops.w8a8_gemm_quant_out(q.reshape(-1, self.in_features).contiguous(),
                                            s.reshape(-1).float().contiguous(), self.weight, self.weight_scale, bias,
                                            dtype, True)
        return qo.reshape(*lead, self.out_features), so.reshape(lead)

    @torch.no_grad()
    def quantized_output(self, x):
        """``(int8 codes, scale)`` of the fake-quantized output (``quantize_output=True``): the codes
        and per-token scale of the reference's output fake quant (``fake_quant.py:77-82``), from the
        GEMM epilogue, for consumers that take quantized q/k/v (the ``return_scale`` form)."""
        _require_gpu(x, "SmoothQuantLinear")
        if self.output_quant_name == "none":
            raise RuntimeError("quantized_output needs quantize_output=True")
        if not self._w8a8:
            y = self._linear_any_width(x)
            return _row_codes(y.reshape(-1, self.out_features).contiguous(), self.activation_bits)
        fake, q, s = self._input_codes(x)
        if self._fused_output_quant(x, fake):
            return self._output_codes(q, s, x.dtype)
        return ops.quant_per_token_i8(self._linear(x, fake, q, s).contiguous(), True)

    @staticmethod
    def from_float(module, weight_bits=8, activation_bits=8, act_quant="per_token", quantize_output=False,
                   scale_rule="fake"):
        assert isinstance(module, nn.Linear)
        new = SmoothQuantLinear(module.in_features, module.out_features, module.bias is not None,
                                weight_bits=weight_bits, activation_bits=activation_bits, act_quant=act_quant,
                                quantize_output=quantize_output, dtype=module.weight.dtype,
                                scale_rule=scale_rule)
        new = new.to(device=module.weight.device)
        if new.weight_bits < 16:
            _require_gpu(module.weight, "SmoothQuantLinear.from_float")
            w = module.weight.detach().contiguous()
            if new.weight_bits == 8:
                q, s32, _ = ops.w8_quantize_per_channel(w, scale_rule)
            else:
                if w.dtype not in _FAKE_DTYPES:
                    raise NotImplementedError("the fake-quant rule takes fp16 or bf16 weights")
                q, s32 = ops.fake_quant_rows(w, new.weight_bits)
            new.weight = q
            new.weight_scale = s32
        else:
            new.weight = module.weight.detach().clone()
        if module.bias is not None:
            new.bias = module.bias.detach().clone()
        return new

    def __repr__(self):
        return (f"SmoothQuantLinear({self.in_features}, {self.out_features}, "
                f"bias={self.bias is not None}, weight_bits={self.weight_bits}, "
                f"activation_bits={self.activation_bits}, weight_quant={self.weight_quant_name}, "
                f"act_quant={self.act_quant_name}, output_quant={self.output_quant_name})")


def _is_silu(act_fn) -> bool:
    if isinstance(act_fn, nn.SiLU) or act_fn is F.silu:
        return True
    return type(act_fn).__name__ in ("SiLUActivation", "SiLU")


class SmoothQuantPackedMoeExperts(nn.Module):
    """Packed W8A8 experts: ``gate_up_proj`` int8 ``[E,2I,H]``, ``down_proj`` int8 ``[E,H,I]``
    with per-row fp32 scales; ``forward(hidden_states, top_k_index, top_k_weights)`` as
    ``fake_quant.py:166-191``.  The chain runs as routing+quant -> grouped GEMM1 +
    SwiGLU + requant -> grouped GEMM2 -> un-permute (one launch each).  With
    ``scale_rule="fake"`` (default) every step rounds as the reference module does, in the
    weight dtype (fp16 / bf16); ``"export"`` is the fp32-scale runtime chain of
    ``vllm_ascend.patch:2356-2423``.

    W8A8 with a SiLU ``act_fn`` runs the fused chain above.  Other widths (2..8, or >= 16 for
    none) and other activations run the reference's expert loop (``fake_quant.py:166-191``) with
    every linear on the dequantising GEMM and ``act_fn`` applied to its fp16 / bf16 output."""

    def __init__(self, gate_up_proj, down_proj, act_fn, *, weight_bits=8, activation_bits=8, scale_rule="fake"):
        super().__init__()
        self.num_experts = int(gate_up_proj.shape[0])
        self.hidden_dim = int(gate_up_proj.shape[2])
        self.intermediate_dim = int(down_proj.shape[2])
        self.weight_bits = _width(weight_bits, "weight_bits")
        self.activation_bits = _width(activation_bits, "activation_bits")
        if scale_rule not in ("fake", "export"):
            raise ValueError(f"Invalid scale_rule: {scale_rule}")
        # the fused chain: W8A8 with SiLU(gate) * up; anything else takes the expert loop
        self._fused = self.weight_bits == 8 and self.activation_bits == 8 and _is_silu(act_fn)
        if scale_rule == "export" and not self._fused:
            raise ValueError("scale_rule='export' is the W8A8 SiLU runtime chain")
        if gate_up_proj.dtype not in _FAKE_DTYPES and (scale_rule == "fake" or not self._fused):
            raise NotImplementedError("the fake scale rule takes fp16 or bf16 expert weights")
        self.act_fn = act_fn
        self.scale_rule = scale_rule
        _require_gpu(gate_up_proj, "SmoothQuantPackedMoeExperts")
        q13, s13 = self._quant3d(gate_up_proj, scale_rule, self.weight_bits)
        q2, s2 = self._quant3d(down_proj, scale_rule, self.weight_bits)
        self.register_buffer("gate_up_proj", q13)
        self.register_buffer("gate_up_scale", s13)
        self.register_buffer("down_proj", q2)
        self.register_buffer("down_scale", s2)
        self.dtype = gate_up_proj.dtype

    @staticmethod
    def _quant3d(w, rule, bits=8):
        """Per-row codes and fp32 scales of a packed [E, N, K] weight at ``bits`` (>= 16: the weight
        itself and no scale)."""
        e, n, k = w.shape
        w2 = w.detach().reshape(e * n, k).contiguous()
        if bits >= 16:
            return w2.clone().reshape(e, n, k), None
        if bits == 8:
            q, s32, _ = ops.w8_quantize_per_channel(w2, rule)
        else:
            q, s32 = ops.fake_quant_rows(w2, bits)
        return q.reshape(e, n, k), s32.reshape(e, n)

    @staticmethod
    def from_float(module, weight_bits=8, activation_bits=8, scale_rule="fake"):
        return SmoothQuantPackedMoeExperts(module.gate_up_proj.detach(), module.down_proj.detach(), module.act_fn,
                                           weight_bits=weight_bits, activation_bits=activation_bits,
                                           scale_rule=scale_rule)

    def dequantized_weights(self):
        """The fake-quant ``(gate_up_proj, down_proj)`` the reference module holds (``q * s``)."""
        if self.gate_up_scale is None:
            return self.gate_up_proj, self.down_proj
        return ((self.gate_up_proj.float() * self.gate_up_scale[..., None]).to(self.dtype),
                (self.down_proj.float() * self.down_scale[..., None]).to(self.dtype))

    def _codes(self, t2):
        if self.activation_bits >= 16:
            return t2, None
        return _row_codes(t2, self.activation_bits)

    def _forward_expert_loop(self, hidden_states, top_k_index, top_k_weights):
        """The reference's expert loop (``fake_quant.py:166-191``): for each expert hit, gather its
        tokens, quantize, gate/up linear, ``act_fn(gate) * up``, quantize, down linear, scale by
        the routing weight and accumulate into the token rows -- each linear on the dequantising
        GEMM, the elementwise steps in the activation dtype."""
        dt = hidden_states.dtype
        if dt not in _FAKE_DTYPES:
            raise NotImplementedError("the expert loop runs in fp16 or bf16")
        out = torch.zeros_like(hidden_states)
        hits = torch.nn.functional.one_hot(top_k_index, num_classes=self.num_experts).permute(2, 1, 0)
        experts = torch.greater(hits.sum(dim=(-1, -2)), 0).nonzero()
        for row in experts.tolist():
            e = row[0]
            pos, tok = torch.where(hits[e])
            qa, sa = self._codes(hidden_states[tok].contiguous())
            gate_up = ops.dq_linear(qa, sa, self.gate_up_proj[e],
                                    None if self.gate_up_scale is None else self.gate_up_scale[e], None, dt)
            gate, up = gate_up.chunk(2, dim=-1)
            h = self.act_fn(gate) * up
            qh, sh = self._codes(h.contiguous())
            y = ops.dq_linear(qh, sh, self.down_proj[e], None if self.down_scale is None else self.down_scale[e],
                              None, dt)
            y = y * top_k_weights[tok, pos, None]
            out.index_add_(0, tok, y.to(out.dtype))
        return out

    @torch.no_grad()
    def forward(self, hidden_states: torch.Tensor, top_k_index: torch.Tensor,
                top_k_weights: torch.Tensor) -> torch.Tensor:
        _require_gpu(hidden_states, "SmoothQuantPackedMoeExperts")
        if not self._fused:
            return self._forward_expert_loop(hidden_states, top_k_index, top_k_weights)
        rule = "fake" if self.scale_rule == "fake" else "runtime"
        return ops.moe_w8a8_forward(hidden_states.contiguous(), top_k_index, top_k_weights, self.gate_up_proj,
                                    self.gate_up_scale, self.down_proj, self.down_scale,
                                    out_dtype=hidden_states.dtype, rule=rule)

    def __repr__(self):
        return (f"SmoothQuantPackedMoeExperts(num_experts={self.num_experts}, "
                f"hidden_dim={self.hidden_dim}, intermediate_dim={self.intermediate_dim}, "
                f"weight_bits={self.weight_bits}, activation_bits={self.activation_bits})")


# model types quantize_llama_like accepts (fake_quant.py:227-239)
SUPPORTED_MODEL_TYPES = frozenset({"llama", "qwen2", "qwen2_5_vl", "qwen3", "qwen3_moe", "qwen3_vl", "qwen3_5",
                                   "qwen3_5_moe", "qwen3_5_moe_text", "minicpm", "minicpmv"})
# accepted only with ``allow_extension_models=True``: the HF Mixtral / Mistral decoders
# (packed ``mlp.experts`` like qwen3_moe, or a dense MLP), which the reference router rejects
# but its serving runtime routes (``packed_modules_model_mapping``, vllm_ascend.patch:3473-3484)
EXTENSION_MODEL_TYPES = frozenset({"mixtral", "mistral"})


def text_backbone(model):
    """``(root, prefix)`` of the decoder stack, resolved in the order of the reference's
    ``get_text_backbone`` (``algorithm/common/modeling.py``): a text-model adapter, ``llm.model``
    (MiniCPM-V), ``model.language_model`` (Qwen2.5-VL / Qwen3-VL; or its ``.model`` for
    LLaVA-style wrappers), ``language_model``, ``model``, ``model.decoder``, ``transformer``
    (``h``)."""
    tm = getattr(model, "text_model", None)
    if tm is not None:
        if hasattr(getattr(tm, "model", None), "layers"):
            return tm.model, "text_model.model"
        if hasattr(tm, "layers"):
            return tm, "text_model"
    llm = getattr(model, "llm", None)
    if llm is not None and hasattr(getattr(llm, "model", None), "layers"):
        return llm.model, "llm.model"
    inner = getattr(model, "model", None)
    lm = getattr(inner, "language_model", None) if inner is not None else None
    if lm is not None:
        if hasattr(lm, "layers"):
            return lm, "model.language_model"
        if hasattr(getattr(lm, "model", None), "layers"):
            return lm.model, "model.language_model.model"
    if hasattr(getattr(model, "language_model", None), "layers"):
        return model.language_model, "language_model"
    if inner is not None and hasattr(inner, "layers"):
        return inner, "model"
    if inner is not None and hasattr(getattr(inner, "decoder", None), "layers"):
        return inner.decoder, "model.decoder"
    if hasattr(getattr(model, "transformer", None), "h"):
        return model.transformer, "transformer"
    raise NotImplementedError(f"Unsupported model backbone: {type(model)}")


def _layers_of(root):
    return root.layers if hasattr(root, "layers") else root.h


def quantize_llama_like(model, weight_bits=8, activation_bits=8, act_quant="per_token", quantize_bmm_input=True,
                        scale_rule="fake", *, allow_extension_models=False) -> List[str]:
    """Module-swap router (``fake_quant.py:226-438``), per decoder layer:

    * attention: q/k/v (output quant when ``quantize_bmm_input``) and o; for Qwen3.5 and
      Qwen3.5-MoE linear-attention layers ``in_proj_qkv / in_proj_z / in_proj_a / in_proj_b``
      (output quant) and ``out_proj`` instead (``:249-293``);
    * MLP: none for ``qwen3_5`` (its dense MLP stays in floating point, ``:249-293``); the
      Qwen3.5-MoE ``shared_expert`` gate/up/down, ``shared_expert_gate`` and the packed experts
      (``:294-362``); for ``qwen3_moe`` layers with experts, the per-expert linears of an
      ``nn.ModuleList`` or the packed experts (``:363-406``); gate/up/down for every other
      layer, including ``qwen3_moe``'s dense layers (``:407-437``).

    The token-mixer kind of a Qwen3.5 layer is its ``layer_type`` (the attribute the reference
    reads, as named by the transformers it pins) or, on later transformers, ``block_type``.
    Returns the qualified names in the order the reference appends them."""
    model_type = getattr(getattr(model, "config", None), "model_type", None)
    allowed = SUPPORTED_MODEL_TYPES | (EXTENSION_MODEL_TYPES if allow_extension_models else frozenset())
    if model_type not in allowed:
        raise ValueError(f"Unsupported model type: {model_type!r}")
    root, prefix = text_backbone(model)
    names: List[str] = []
    kw = dict(weight_bits=weight_bits, activation_bits=activation_bits, act_quant=act_quant, scale_rule=scale_rule)

    def swap(parent, attr, qualified, qout=False):
        setattr(parent, attr, SmoothQuantLinear.from_float(getattr(parent, attr), quantize_output=qout, **kw))
        names.append(qualified)

    def mixer_kind(layer):
        kind = getattr(layer, "layer_type", None)
        return getattr(layer, "block_type", None) if kind is None else kind

    def attention(layer, lp):
        if model_type in ("qwen3_5", "qwen3_5_moe", "qwen3_5_moe_text") and mixer_kind(layer) == "linear_attention":
            la = layer.linear_attn
            for p in ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b"):
                swap(la, p, f"{lp}.linear_attn.{p}", quantize_bmm_input)
            swap(la, "out_proj", f"{lp}.linear_attn.out_proj")
            return
        for p in ("q_proj", "k_proj", "v_proj"):
            swap(layer.self_attn, p, f"{lp}.self_attn.{p}", quantize_bmm_input)
        swap(layer.self_attn, "o_proj", f"{lp}.self_attn.o_proj")

    def packed_experts(mlp, lp):
        mlp.experts = SmoothQuantPackedMoeExperts.from_float(mlp.experts, weight_bits=weight_bits,
                                                             activation_bits=activation_bits, scale_rule=scale_rule)
        names.append(f"{lp}.mlp.experts.gate_up_proj")
        names.append(f"{lp}.mlp.experts.down_proj")

    for li, layer in enumerate(_layers_of(root)):
        lp = f"{prefix}.layers.{li}"
        attention(layer, lp)
        if model_type == "qwen3_5":
            continue
        mlp = layer.mlp
        if model_type in ("qwen3_5_moe", "qwen3_5_moe_text"):
            for p in ("gate_proj", "up_proj", "down_proj"):
                swap(mlp.shared_expert, p, f"{lp}.mlp.shared_expert.{p}")
            swap(mlp, "shared_expert_gate", f"{lp}.mlp.shared_expert_gate")
            packed_experts(mlp, lp)
        elif model_type in ("qwen3_moe", "mixtral") and hasattr(mlp, "experts"):
            if isinstance(mlp.experts, nn.ModuleList):
                for ei, ex in enumerate(mlp.experts):
                    for p in ("gate_proj", "up_proj", "down_proj"):
                        swap(ex, p, f"{lp}.mlp.experts.{ei}.{p}")
            else:
                packed_experts(mlp, lp)
        else:
            for p in ("gate_proj", "up_proj", "down_proj"):
                swap(mlp, p, f"{lp}.mlp.{p}")
    return names


def quantize_model(model, weight_bits=8, activation_bits=8, weight_quant="per_channel", act_quant="per_token",
                   quantize_bmm_input=True, scale_rule="fake", *, allow_extension_models=False) -> List[str]:
    """``fake_quant.py:441-457``."""
    if weight_quant != "per_channel":
        raise ValueError(f"Invalid weight_quant: {weight_quant}")
    return quantize_llama_like(model, weight_bits=weight_bits, activation_bits=activation_bits,
                               act_quant=act_quant, quantize_bmm_input=quantize_bmm_input, scale_rule=scale_rule,
                               allow_extension_models=allow_extension_models)


# ------------------------------------------------------------------ smoothing (smooth.py, calibration.py)
def _colmax_of(tensors, k: int) -> torch.Tensor:
    cm = None
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError("SmoothQuant smoothing runs on the GPU only; move the model to the GPU first")
        cm = ops.colmax_abs(t.detach().reshape(-1, k), cm)
    return cm


def _scales_for(weights, act_scales: torch.Tensor, alpha: float, like: torch.Tensor) -> torch.Tensor:
    k = act_scales.numel()
    cm = _colmax_of(weights, k)
    a = act_scales.detach().to(device=like.device, dtype=torch.float32).reshape(-1).contiguous()
    return ops.smooth_scales(a, cm, alpha, like.dtype)


@torch.no_grad()
def compute_smooth_scales(fcs, act_scales: torch.Tensor, alpha: float = 0.5) -> torch.Tensor:
    """``_compute_smooth_scales`` (``smooth.py:7-25``) on the GPU: ``(a^alpha / w^(1-alpha)).clamp(1e-5)``
    in the weight dtype, ``a`` the activation statistic cast to that dtype and ``w_j = max_n |W_nj|``
    over every fc sharing the norm (clamped at 1e-5).  Same checks as the reference (``AssertionError``
    on a non-Linear or a width mismatch)."""
    if not isinstance(fcs, (list, tuple)):
        fcs = [fcs]
    for fc in fcs:
        assert isinstance(fc, nn.Linear)
        assert fc.in_features == act_scales.numel()
    return _scales_for([fc.weight for fc in fcs], act_scales, alpha, fcs[0].weight)


def _norm_weight(ln):
    if not hasattr(ln, "weight") or ln.weight is None:
        raise TypeError(f"SmoothQuant requires a norm module with a learnable weight; got {type(ln)}")
    return ln.weight


@torch.no_grad()
def smooth_ln_fcs_llama_like(ln, fcs, act_scales, alpha=0.5):
    """``smooth.py:91-101``: ``ln.weight /= s`` and every fc weight ``*= s`` along its input columns,
    each product / quotient rounded to the weight dtype (the in-place half ops of the reference)."""
    w = _norm_weight(ln)
    assert w.numel() == act_scales.numel()
    if not isinstance(fcs, (list, tuple)):
        fcs = [fcs]
    s = compute_smooth_scales(fcs, act_scales, alpha)
    ops.scale_columns_(w.data, s.to(w.dtype), divide=True)
    for fc in fcs:
        ops.scale_columns_(fc.weight.data, s)


def _qwen3_5_norm_update(ln, s):
    """Qwen3.5 norms scale by ``1 + weight``: ``weight = (1 + weight) / s - 1`` in float64, cast back
    (``smooth.py:104-117``)."""
    w = ln.weight.data
    ln.weight.data = ((1.0 + w.to(torch.float64)) / s.to(torch.float64) - 1.0).to(w.dtype)


@torch.no_grad()
def smooth_ln_fcs_qwen3_5(ln, fcs, act_scales, alpha=0.5):
    """``smooth.py:104-117``: the Qwen3.5 ``(1 + w)`` norm update, fc weights ``*= s``."""
    assert _norm_weight(ln).numel() == act_scales.numel()
    s = compute_smooth_scales(fcs, act_scales, alpha)
    _qwen3_5_norm_update(ln, s)
    for fc in fcs:
        ops.scale_columns_(fc.weight.data, s)


def _experts_packed(experts) -> bool:
    return not isinstance(experts, nn.ModuleList)


@torch.no_grad()
def smooth_qwen3_moe_ffn(ln, mlp, act_scales, alpha=0.5):
    """``smooth.py:147-168``: one scale over the router and every expert's gate/up (per-expert
    linears or the packed ``gate_up_proj [E, 2I, H]``); ``ln /= s``, all of them ``*= s``."""
    assert _norm_weight(ln).numel() == act_scales.numel()
    k = act_scales.numel()
    ws = [mlp.gate.weight]
    if _experts_packed(mlp.experts):
        ws.append(mlp.experts.gate_up_proj)
    else:
        for ex in mlp.experts:
            ws += [ex.gate_proj.weight, ex.up_proj.weight]
    for w in ws:
        assert w.shape[-1] == k
    s = _scales_for(ws, act_scales, alpha, mlp.gate.weight)
    ops.scale_columns_(ln.weight.data, s.to(ln.weight.dtype), divide=True)
    for w in ws:
        ops.scale_columns_(w.data, s.to(w.dtype))


@torch.no_grad()
def smooth_qwen3_5_moe_ffn(ln, mlp, act_scales, alpha=0.5):
    """``smooth.py:120-144``: one scale over the shared expert's gate/up, ``shared_expert_gate``, the
    router and the packed experts' ``gate_up_proj``; the Qwen3.5 norm update; all of them ``*= s``."""
    assert _norm_weight(ln).numel() == act_scales.numel()
    k = act_scales.numel()
    ws = [mlp.shared_expert.gate_proj.weight, mlp.shared_expert.up_proj.weight, mlp.shared_expert_gate.weight,
          mlp.gate.weight, mlp.experts.gate_up_proj]
    for w in ws:
        assert w.shape[-1] == k
    s = _scales_for(ws, act_scales, alpha, mlp.shared_expert.gate_proj.weight)
    _qwen3_5_norm_update(ln, s)
    for w in ws:
        ops.scale_columns_(w.data, s.to(w.dtype))


SMOOTH_MODEL_TYPES = SUPPORTED_MODEL_TYPES


@torch.no_grad()
def smooth_lm(model, scales, alpha=0.5):
    """``smooth_lm`` (``smooth.py:171-245``): per decoder layer, smooth the attention input norm into
    q/k/v (Qwen3.5 linear-attention layers: ``in_proj_qkv/z/a/b``) and the MLP input norm into
    gate/up (or the MoE router and experts), keyed by the qualified names of ``get_act_scales``."""
    model_type = getattr(getattr(model, "config", None), "model_type", None)
    if model_type not in SMOOTH_MODEL_TYPES:
        raise NotImplementedError(f"Unsupported SmoothQuant model type: {model_type!r}")
    root, prefix = text_backbone(model)
    qwen35 = model_type in ("qwen3_5", "qwen3_5_moe", "qwen3_5_moe_text")
    for li, layer in enumerate(_layers_of(root)):
        lp = f"{prefix}.layers.{li}"
        if qwen35:
            if getattr(layer, "layer_type", None) == "linear_attention":
                la = layer.linear_attn
                fcs = [la.in_proj_qkv, la.in_proj_z, la.in_proj_a, la.in_proj_b]
                key = lp + ".linear_attn.in_proj_qkv"
            else:
                fcs = [layer.self_attn.q_proj, layer.self_attn.k_proj, layer.self_attn.v_proj]
                key = lp + ".self_attn.q_proj"
            smooth_ln_fcs_qwen3_5(layer.input_layernorm, fcs, scales[key], alpha)
            if model_type == "qwen3_5":
                smooth_ln_fcs_qwen3_5(layer.post_attention_layernorm, [layer.mlp.gate_proj, layer.mlp.up_proj],
                                      scales[lp + ".mlp.gate_proj"], alpha)
            else:
                smooth_qwen3_5_moe_ffn(layer.post_attention_layernorm, layer.mlp,
                                       scales[lp + ".mlp.shared_expert.gate_proj"], alpha)
            continue
        qkv = [layer.self_attn.q_proj, layer.self_attn.k_proj, layer.self_attn.v_proj]
        smooth_ln_fcs_llama_like(layer.input_layernorm, qkv, scales[lp + ".self_attn.q_proj"], alpha)
        if model_type == "qwen3_moe" and hasattr(layer.mlp, "experts"):
            smooth_qwen3_moe_ffn(layer.post_attention_layernorm, layer.mlp, scales[lp + ".mlp.gate"], alpha)
        else:
            smooth_ln_fcs_llama_like(layer.post_attention_layernorm, [layer.mlp.gate_proj, layer.mlp.up_proj],
                                     scales[lp + ".mlp.gate_proj"], alpha)


_MASKED_CALIBRATION = {"qwen2_5_vl", "qwen3_vl", "qwen3_moe", "qwen3_5", "qwen3_5_moe", "qwen3_5_moe_text"}


@torch.no_grad()
def get_act_scales(model, calibration_batches, device=None):
    """``get_act_scales`` (``calibration.py:27-58``): the per-input-channel ``max |x|`` of every
    ``nn.Linear``'s input over all calibration tokens, keyed by qualified name, fp32 on the host.

    The statistics are kept on the GPU and updated by the column abs-max kernel after each linear's
    forward; ``calibration_batches`` yields ``(token_ids, labels)`` pairs.  The forward passes
    ``use_cache=False`` (and an all-ones attention mask for the model types the reference gives one).
    ``device`` is accepted for the reference's signature: the tokens go to the embedding's device."""
    del device
    model.eval()
    root, prefix = text_backbone(model)
    emb = getattr(getattr(root, "embed_tokens", None), "weight", None)
    in_dev = emb.device if emb is not None else next(model.parameters()).device
    stats = {}

    def hook(_m, inputs, _out, name):
        x = inputs[0] if isinstance(inputs, tuple) else inputs
        stats[name] = ops.colmax_abs(x.detach(), stats.get(name))

    handles = []
    for n, m in root.named_modules():
        if isinstance(m, nn.Linear):
            q = f"{prefix}.{n}" if n else prefix
            handles.append(m.register_forward_hook(partial(hook, name=q)))
    mtype = getattr(getattr(model, "config", None), "model_type", None)
    try:
        for ids, _labels in calibration_batches:
            ids = ids.to(in_dev)
            kw = {"attention_mask": torch.ones_like(ids, dtype=torch.long)} if mtype in _MASKED_CALIBRATION else {}
            model(input_ids=ids, use_cache=False, **kw)
    finally:
        for h in handles:
            h.remove()
    return {k: v.cpu() for k, v in stats.items()}
