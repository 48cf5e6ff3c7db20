"""Runtime operator contract of the reference's deployed W8A8 path, on the gfx950 kernels.

``W8A8DynamicLinearMethod`` replaces ``AscendW8A8DynamicLinearMethod`` as patched by
MindPipe (``acceleration/runtime_patches/vllm_ascend.patch:3935-4033``): per-token
dynamic int8 quant (fp32 scale, the ``npu_dynamic_quant`` contract) then the int8
GEMM with the per-token x per-channel epilogue (``npu_quant_matmul``).
``fused_experts_w8a8`` replaces the MoE expert chain of ``_run_expert_tile``
(``vllm_ascend.patch:2356-2423``) and ``W8A8DynamicFusedMoEMethod`` the fused-MoE method's weight
processing and ``apply`` (``:4278-4482``).  ``add_rms_norm_forward`` replaces the
add-RMSNorm(-dynamic-quant) step in front of a W8A8 linear
(``_addrmsnorm_forward_oot``, ``vllm_ascend.patch:740-792``), and
``prepare_dense_mlp_w8a8`` / ``dense_mlp_w8a8`` the chunked dense-MLP chain
(``vllm.patch:883-1037``, weight split ``vllm_ascend.patch:4149-4277``).  Layer attributes keep the reference's names
(``weight``, ``weight_scale``, ``weight_offset``, ``weight_scale_fp32``,
``_ascend_quant_config``); the weight stays ``[N, K]`` (the kernel reads that layout
directly, so no transpose or NZ cast is needed).
"""
from __future__ import annotations

import os
from typing import Optional, Tuple, Union

import torch

from . import ops

__all__ = ["W8A8DynamicLinearMethod", "W8A8DynamicFusedMoEMethod", "fused_experts_w8a8", "grouped_apply_mlp_w8a8",
           "layout_conversions", "dynamic_quant",
           "add_rms_norm_forward", "prepare_dense_mlp_w8a8", "dense_mlp_w8a8"]


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


_LAYOUT_CONVERSIONS = [0]


def layout_conversions() -> int:
    """How many weight tensors ``fused_experts_w8a8`` / ``grouped_apply_mlp_w8a8`` have re-laid in
    place so far (each at most once: afterwards the tensor's own strides give the kernel view)."""
    return _LAYOUT_CONVERSIONS[0]


def _kernel_view(w: torch.Tensor, name: str) -> torch.Tensor:
    """The kernel layout ``[E, N, K]`` (each output row's K bytes contiguous, the int8 MFMA
    operand) of a runtime-layout expert weight ``w [E, K, N]`` (``vllm_ascend.patch:2278-2291``).

    After ``W8A8DynamicFusedMoEMethod.process_weights_after_loading`` the layer's ``[E, K, N]``
    weight is a strided view of ``[E, N, K]`` storage, so this is ``w.transpose(1, 2)`` with no
    copy.  A contiguous ``[E, K, N]`` tensor (laid out by some other loader) has its storage
    re-laid once, in place: its values, shape, dtype and device are unchanged and its strides
    become the kernel view's, so later calls find that view; nothing is cached beside it."""
    if w.dim() != 3 or w.dtype != torch.int8:
        raise ValueError(f"{name} must be an int8 [E, K, N] expert weight, got {w.dtype} {tuple(w.shape)}")
    kv = w.transpose(1, 2)
    if kv.is_contiguous():
        return kv
    with torch.no_grad():
        w.data = w.data.transpose(1, 2).contiguous().transpose(1, 2)
    _LAYOUT_CONVERSIONS[0] += 1
    return w.transpose(1, 2)


def _expert_weights(w1, w1_scale, w2, w2_scale, hidden):
    """Kernel views ``w13 [E, 2I, H]`` / ``w2 [E, H, I]`` of the runtime-layout weights
    ``w1 [E, H, 2I]`` / ``w2 [E, I, H]``, and fp32 per-row scales ``[E, 2I]`` / ``[E, H]`` from
    scales of any float dtype shaped ``[E, N]`` or ``[E, N, 1]``."""
    if w1.dim() != 3 or w2.dim() != 3 or w1.shape[1] != hidden or w2.shape[2] != hidden or \
            w1.shape[0] != w2.shape[0] or w1.shape[2] != 2 * w2.shape[1]:
        raise ValueError(f"expected w1 [E, {hidden}, 2I] and w2 [E, I, {hidden}], got {tuple(w1.shape)} "
                         f"and {tuple(w2.shape)}")
    k1, k2 = _kernel_view(w1, "w1"), _kernel_view(w2, "w2")
    e = w1.shape[0]
    s1 = w1_scale.reshape(e, -1).to(torch.float32).contiguous()
    s2 = w2_scale.reshape(e, -1).to(torch.float32).contiguous()
    return k1, s1, k2, s2


def fused_experts_w8a8(hidden_states: torch.Tensor, w1: torch.Tensor, w1_scale: torch.Tensor, w2: torch.Tensor,
                       w2_scale: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor,
                       row_idx: Optional[torch.Tensor] = None, use_int8_w8a8: bool = True,
                       pertoken_scale: Optional[torch.Tensor] = None, expert_map: Optional[torch.Tensor] = None,
                       output_dtype: Optional[torch.dtype] = None, **_unused) -> torch.Tensor:
    """The runtime's ``fused_experts(hidden_states, w1, w1_scale, w2, w2_scale, topk_weights,
    topk_ids, row_idx, use_int8_w8a8=True, pertoken_scale, expert_map, ..., output_dtype)``
    (``vllm_ascend.patch:4447-4468``) on the gfx950 chain: routing quant -> grouped GEMM1 +
    SwiGLU + requant -> grouped GEMM2 -> weighted un-permute.

    * ``w1`` int8 ``[E, H, 2I]`` (gate columns first) and ``w2`` int8 ``[E, I, H]``: the runtime's
      loaded layout, read through the kernel view of ``_kernel_view``;
      ``w1_scale [E, 2I]`` / ``w2_scale [E, H]`` in any float dtype.
    * ``pertoken_scale``: ``hidden_states`` is already int8 with these fp32 per-token scales
      (routed without re-quantizing); ``output_dtype`` then defaults to fp16.
    * ``expert_map`` (expert parallelism: global -> local id, -1 = not on this rank): ids are
      mapped and assignments to other ranks contribute nothing.
    * ``row_idx`` is accepted for signature compatibility; the routing kernel builds its own.
    """
    if not use_int8_w8a8:
        raise NotImplementedError("fused_experts_w8a8 is the int8 W8A8 path")
    k1, s1, k2, s2 = _expert_weights(w1, w1_scale, w2, w2_scale, hidden_states.shape[-1])
    ids = topk_ids.to(torch.int32)
    if expert_map is not None:
        ids = expert_map.to(device=ids.device, dtype=torch.int32)[ids.long()]
    if pertoken_scale is not None:
        return ops.moe_w8a8_forward(hidden_states.contiguous(), ids.contiguous(), topk_weights, k1, s1, k2, s2,
                                    out_dtype=output_dtype or torch.float16, rule="runtime",
                                    x_scale=pertoken_scale.reshape(-1).to(torch.float32).contiguous())
    return ops.moe_w8a8_forward(hidden_states.contiguous(), ids.contiguous(), topk_weights, k1, s1, k2, s2,
                                out_dtype=output_dtype or hidden_states.dtype, rule="runtime")


def grouped_apply_mlp_w8a8(hidden_states: torch.Tensor, w1: torch.Tensor, w1_scale: torch.Tensor, w2: torch.Tensor,
                           w2_scale: torch.Tensor, group_list: torch.Tensor, group_list_type: int = 0,
                           dynamic_scale: Optional[torch.Tensor] = None,
                           output_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """The runtime's ``quant_apply_mlp`` on already-permuted rows (``vllm_ascend.patch:2895-2964``):
    ``hidden_states [R, H]`` grouped by expert with ``group_list`` cumulative endpoints
    (``group_list_type=0``) or raw counts (``1``) (``:2015-2031``); quantized here unless
    ``dynamic_scale`` marks it as int8 codes.  Weights in the runtime layout as for
    ``fused_experts_w8a8``.  GEMM1 + SwiGLU + requant, then GEMM2 with the per-token scale,
    output ``output_dtype`` (default fp16; the reference's default is the down scale's dtype).
    There is no 10240-column limit (``_can_use_fused_swiglu_quant``)."""
    k1, s1, k2, s2 = _expert_weights(w1, w1_scale, w2, w2_scale, hidden_states.shape[-1])
    offsets = ops.group_offsets_from_list(group_list.to(hidden_states.device), group_list_type)
    if dynamic_scale is None:
        qx, sx = dynamic_quant(hidden_states)
    else:
        qx, sx = hidden_states.contiguous(), dynamic_scale.reshape(-1).to(torch.float32).contiguous()
    inter = k2.shape[2]
    qh, sh = ops.moe_gmm1_swiglu_quant(qx, sx, k1, s1, offsets, inter)
    return ops.moe_gmm2(qh, sh, k2, s2, offsets, output_dtype or torch.float16)


class W8A8DynamicFusedMoEMethod:
    """Replaces ``AscendW8A8DynamicFusedMoEMethod`` (``vllm_ascend.patch:4278-4482``): weight
    processing after loading, and ``apply`` on already-selected experts.

    ``process_weights_after_loading``: the checkpoint loads ``w13_weight [E, 2I, H]`` and
    ``w2_weight [E, H, I]``; the reference transposes them to ``[E, H, 2I]`` / ``[E, I, H]`` for
    its NPU kernels.  Here the layer's tensors take that shape as strided views of the loaded
    storage (no copy, no second buffer): the gfx950 grouped GEMMs read the loaded rows directly,
    and ``fused_experts_w8a8`` recovers them from the view.  Scales are flattened to ``[E, N]``
    with fp32 copies ``w13_weight_scale_fp32`` / ``w2_weight_scale_fp32``, offsets to ``[E, N]``,
    under the reference's attribute names."""

    def __init__(self, in_dtype: torch.dtype = torch.float16):
        self.transpose_weight = True
        self.in_dtype = in_dtype

    def process_weights_after_loading(self, layer) -> None:
        if self.transpose_weight:
            layer.w13_weight.data = layer.w13_weight.data.transpose(1, 2)
            layer.w2_weight.data = layer.w2_weight.data.transpose(1, 2)
        for name in ("w13", "w2"):
            sc = getattr(layer, f"{name}_weight_scale")
            sc.data = sc.data.view(sc.data.shape[0], -1)
            setattr(layer, f"{name}_weight_scale_fp32", sc.data.to(torch.float32))
            off = getattr(layer, f"{name}_weight_offset", None)
            if off is not None:
                off.data = off.data.view(off.data.shape[0], -1)

    def apply(self, layer, x: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor,
              expert_map: Optional[torch.Tensor] = None, pertoken_scale: Optional[torch.Tensor] = None,
              row_idx: Optional[torch.Tensor] = None, **_unused) -> torch.Tensor:
        """The expert chain of ``apply`` once experts are selected (``:4430-4468``): fp32 weight
        scales under fp16 models, the stored scales otherwise; ``topk_weights`` cast to the model
        dtype; output in the model dtype."""
        if self.in_dtype == torch.float16:
            w1_scale, w2_scale = layer.w13_weight_scale_fp32, layer.w2_weight_scale_fp32
        else:
            w1_scale, w2_scale = layer.w13_weight_scale, layer.w2_weight_scale
        return fused_experts_w8a8(hidden_states=x, w1=layer.w13_weight, w1_scale=w1_scale, w2=layer.w2_weight,
                                  w2_scale=w2_scale, topk_weights=topk_weights.to(self.in_dtype), topk_ids=topk_ids,
                                  row_idx=row_idx, use_int8_w8a8=True, pertoken_scale=pertoken_scale,
                                  expert_map=expert_map, output_dtype=self.in_dtype)


# ---------------------------------------------------------------- add + RMSNorm (+ dynamic quant)
def _env_int(name: str, default: int) -> int:
    try:
        return int(os.getenv(name, str(default)))
    except ValueError:
        return default


def _quant_method_of(layer):
    qm = getattr(layer, "quant_method", None)
    return getattr(qm, "quant_method", qm)


def _is_w8a8_dynamic_linear(layer) -> bool:
    return isinstance(_quant_method_of(layer), W8A8DynamicLinearMethod)


def _should_use_w8a8_dynamic_fusion(layer, x: torch.Tensor) -> bool:
    """Token window of ``vllm_ascend.patch:720-738`` (same environment names and defaults,
    ``:505-512``:
    ``MINDPIPE_W8A8_DYNAMIC_RMSNORM_QUANT_MAX_TOKENS`` 256, ``..._MIN_TOKENS`` 0; a maximum
    <= 0 removes the upper bound).  Here the fused and unfused paths give the same bits,
    so the window only chooses the kernel count."""
    if not _is_w8a8_dynamic_linear(layer):
        return False
    max_tokens = _env_int("MINDPIPE_W8A8_DYNAMIC_RMSNORM_QUANT_MAX_TOKENS", 256)
    min_tokens = max(0, _env_int("MINDPIPE_W8A8_DYNAMIC_RMSNORM_QUANT_MIN_TOKENS", 0))
    tokens = x.numel() // x.shape[-1]
    if max_tokens <= 0:
        return tokens >= min_tokens
    return min_tokens <= tokens <= max_tokens


def add_rms_norm_forward(norm, x: torch.Tensor, residual: Optional[torch.Tensor], layer=None):
    """``_addrmsnorm_forward_oot(self, x, residual, layer)`` (``vllm_ascend.patch:740-792``).

    ``norm`` carries ``weight`` and ``variance_epsilon`` (an RMSNorm module).  When the next
    linear ``layer`` is a W8A8 dynamic linear inside the token window, returns
    ``((int8 codes, fp32 scale), residual_sum)`` for its ``apply`` (the
    ``npu_add_rms_norm_dynamic_quant`` branch); otherwise ``(normalised x, residual_sum)`` (the
    ``npu_add_rms_norm`` branch).  With ``residual=None`` this is a plain RMSNorm and the
    returned residual is ``x`` itself (the first layer of vLLM's decoder).
    """
    eps = float(getattr(norm, "variance_epsilon", getattr(norm, "eps", 1e-6)))
    weight = norm.weight
    mp = torch.ops.mindpipe_amd
    if layer is not None and _should_use_w8a8_dynamic_fusion(layer, x):
        if residual is None:
            q, s = mp.rms_norm_dynamic_quant(x, weight, eps)
            return (q, s), x
        q, s, rsum = mp.add_rms_norm_dynamic_quant(x, residual, weight, eps)
        return (q, s), rsum
    if residual is None:
        y, _, _, _ = ops.add_rms_norm_quant(x, None, weight, eps, quant=False)
        return y, x
    y, rsum = mp.add_rms_norm(x, residual, weight, eps)
    return y, rsum


# ---------------------------------------------------------------- dense MLP chain
_OFFSETS = {}


def _group_offsets(tokens: int, device) -> torch.Tensor:
    """Cumulative group boundaries ``[0, T]`` of a dense call (one group of all tokens),
    cached per device and T so that graph capture records no host copy."""
    key = (str(device), tokens)
    t = _OFFSETS.get(key)
    if t is None:
        t = torch.tensor([0, tokens], dtype=torch.int64, device=device)
        _OFFSETS[key] = t
    return t


def prepare_dense_mlp_w8a8(gate_up, down, chunks: int = 1) -> None:
    """Split a W8A8 ``gate_up`` / ``down`` pair into the chunk buffers of
    ``_prepare_qwen2_gate_up_chunked_w8a8`` / ``_prepare_qwen2_down_chunked_w8a8``
    (``vllm_ascend.patch:4149-4277``; same attribute names).  ``gate_up.weight`` is int8
    ``[2I, H]`` (gate rows first), ``down.weight`` int8 ``[H, I]``, each with
    ``weight_scale_fp32`` per output row (``process_weights_after_loading``).  Chunk ``c``
    holds gate rows ``[c*cs, (c+1)*cs)`` and the matching up rows as ``[1, 2cs, H]`` (the
    grouped kernel's ``[E, 2I, H]`` layout with one group); the down chunks are the matching
    column slices ``[H, cs]`` with the down scale rounded to bf16 (``:4262-4264``; the
    single-chunk path keeps the fp32 scale, ``vllm.patch:1003-1037``).  There is no
    10240-column limit here, so ``chunks=1`` is the
    fast choice; larger counts reproduce the reference's per-chunk requantisation.
    """
    w, sc = gate_up.weight.data, gate_up.weight_scale_fp32
    inter = w.shape[0] // 2
    if w.shape[0] % 2 or inter % chunks:
        raise ValueError(f"gate_up rows {w.shape[0]} do not split into {chunks} chunks")
    if down.weight.shape[1] != inter:
        raise ValueError("down.weight must be [H, I]")
    cs = inter // chunks
    for idx in range(chunks):
        rows = torch.cat([torch.arange(idx * cs, (idx + 1) * cs), torch.arange(inter + idx * cs, inter + (idx + 1) * cs)])
        rows = rows.to(w.device)
        setattr(gate_up, f"_mindpipe_chunked_gate_up_weight_{idx}", w.index_select(0, rows).unsqueeze(0).contiguous())
        setattr(gate_up, f"_mindpipe_chunked_gate_up_scale_{idx}",
                sc.index_select(0, rows).reshape(1, 2 * cs).to(torch.float32).contiguous())
    dw = down.weight.data
    down._mindpipe_chunked_down_weight = torch.stack([dw[:, i * cs:(i + 1) * cs] for i in range(chunks)]).contiguous()
    down._mindpipe_chunked_down_scale_bf16 = down.weight_scale_fp32.to(torch.bfloat16).contiguous()
    down._mindpipe_chunked_down_scale_fp32 = (down.weight_scale_fp32 if chunks == 1 else
                                              down._mindpipe_chunked_down_scale_bf16).to(torch.float32).contiguous()
    for layer, kind in ((gate_up, "gate_up"), (down, "down")):
        layer._mindpipe_qwen2_mlp_chunked_kind = kind
        layer._mindpipe_qwen2_mlp_chunk_count = chunks
        layer._mindpipe_qwen2_mlp_chunk_size = cs


def dense_mlp_w8a8(gate_up, down, x: Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]) -> torch.Tensor:
    """``_mindpipe_forward_chunked_mlp_w8a8`` (``vllm.patch:883-937``; one chunk
    ``:1003-1037``) on the gfx950 kernels.

    ``x`` is activations ``[T, H]`` (quantized here, fp32 per-token scale) or a pre-quantized
    ``(int8 [T, H], scale)`` tuple (from ``add_rms_norm_forward``).  Each chunk runs the grouped
    GEMM1 + SwiGLU + requant kernel with one group of all tokens, then the int8 down GEMM on the
    chunk's columns; chunk outputs are summed in fp32 and rounded once to the output dtype
    (``x.dtype``, or ``down.params_dtype`` / fp16 for a tuple input, as in
    ``_mindpipe_chunked_mlp_output_dtype``).
    """
    chunks = int(getattr(gate_up, "_mindpipe_qwen2_mlp_chunk_count"))
    cs = int(gate_up._mindpipe_qwen2_mlp_chunk_size)
    if isinstance(x, tuple):
        qx, sx = x
        out_dtype = getattr(down, "params_dtype", torch.float16)
        lead = qx.shape[:-1]
        qx = qx.reshape(-1, qx.shape[-1]).contiguous()
        sx = sx.flatten().to(torch.float32).contiguous()
    else:
        out_dtype = x.dtype
        lead = x.shape[:-1]
        qx, sx = dynamic_quant(x.reshape(-1, x.shape[-1]))
    offsets = _group_offsets(qx.shape[0], qx.device)
    w13 = [getattr(gate_up, f"_mindpipe_chunked_gate_up_weight_{i}") for i in range(chunks)]
    s13 = [getattr(gate_up, f"_mindpipe_chunked_gate_up_scale_{i}") for i in range(chunks)]
    out = torch.ops.mindpipe_amd.dense_mlp_w8a8(qx, sx, offsets, w13, s13, down._mindpipe_chunked_down_weight,
                                                down._mindpipe_chunked_down_scale_fp32, cs, out_dtype)
    return out.reshape(*lead, out.shape[-1])
