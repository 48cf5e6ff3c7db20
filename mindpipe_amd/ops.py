"""Torch-facing operators over the C ABI.

Each function validates device/dtype/shape/contiguity the way the reference's
torch extension does with ``TORCH_CHECK`` (``aclnn_grouped_swiglu_out_bridge.cpp:97-109,163-202``),
allocates outputs with the caching allocator, and launches on the current HIP
stream.  The functions are also registered as ``torch.ops.mindpipe_amd.*``
custom ops with fake (meta) implementations so that ``torch.compile`` and graph
capture see shapes without running kernels (the pattern of the reference's
``torch.ops.vllm.mindpipe_qwen2_grouped_swiglu_loop_out`` registration,
``vllm.patch:171-228,291-306``).
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import torch

from . import _lib
from ._lib import MP_BF16, MP_F16, MP_F32, MP_I8, MP_SCALE_FAKE, MP_SCALE_FP32

_DT = {torch.float16: MP_F16, torch.bfloat16: MP_BF16, torch.float32: MP_F32}


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _need(t: torch.Tensor, name: str, dtype=None, ndim=None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be on the GPU (mindpipe_amd has no CPU path)")
    if dtype is not None and t.dtype not in (dtype if isinstance(dtype, tuple) else (dtype,)):
        raise RuntimeError(f"{name} has dtype {t.dtype}, expected {dtype}")
    if ndim is not None and t.dim() != ndim:
        raise RuntimeError(f"{name} must be {ndim}-D, got shape {tuple(t.shape)}")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def _dev(t: torch.Tensor):
    return torch.cuda.device(t.device)


# ---------------------------------------------------------------- W4
def w4_quantize_awq(w: torch.Tensor, group_size: int = 128, zero_point: bool = True,
                    return_deq: bool = True):
    """AWQ ``pseudo_quantize_tensor`` on the GPU, in the arithmetic of ``w``'s dtype (fp16 or
    bf16): returns ``(packed, scales, zeros, w_deq)`` with scales / zeros / w_deq in that dtype."""
    _need(w, "w", (torch.float16, torch.bfloat16), 2)
    n, k = w.shape
    g = group_size if (group_size > 0 and k % group_size == 0) else k
    packed = torch.empty((n, (k + 7) // 8), dtype=torch.int32, device=w.device)
    scales = torch.empty((n, k // g), dtype=w.dtype, device=w.device)
    zeros = torch.empty_like(scales) if zero_point else None
    deq = torch.empty_like(w) if return_deq else None
    with _dev(w):
        _lib.check(_lib.load().mp_w4_quantize_awq(
            w.data_ptr(), _DT[w.dtype], n, k, group_size, int(zero_point), packed.data_ptr(), scales.data_ptr(),
            _ptr(zeros), _ptr(deq), _stream()), "mp_w4_quantize_awq")
    return packed, scales, zeros, deq


def awq_pseudo_quantize(w: torch.Tensor, n_bit: int, group_size: int = 128, zero_point: bool = True):
    """AWQ ``pseudo_quantize_tensor`` at any code width ``n_bit`` (1..8; 2..8 without a zero point) in
    the arithmetic of ``w``'s dtype: returns ``(scales, zeros, w_deq)`` (zeros ``None`` when symmetric)."""
    _need(w, "w", (torch.float16, torch.bfloat16), 2)
    n, k = w.shape
    g = group_size if (group_size > 0 and k % group_size == 0) else k
    scales = torch.empty((n, k // g), dtype=w.dtype, device=w.device)
    zeros = torch.empty_like(scales) if zero_point else None
    deq = torch.empty_like(w)
    with _dev(w):
        _lib.check(_lib.load().mp_awq_pseudo_quantize(
            w.data_ptr(), _DT[w.dtype], n, k, group_size, int(zero_point), int(n_bit), scales.data_ptr(),
            _ptr(zeros), deq.data_ptr(), _stream()), "mp_awq_pseudo_quantize")
    return scales, zeros, deq


def w4_quantize_gptq_rtn(w: torch.Tensor, group_size: int = 128):
    """GPTQ symmetric RTN group quantizer: returns ``(int_weight int8, packed int32, scale fp16)``."""
    _need(w, "w", (torch.float32, torch.float16, torch.bfloat16), 2)
    n, k = w.shape
    g = group_size if group_size > 0 else k
    if k % g:
        raise ValueError("group_size must divide in_features")
    iw = torch.empty((n, k), dtype=torch.int8, device=w.device)
    packed = torch.empty((n, (k + 7) // 8), dtype=torch.int32, device=w.device)
    scale = torch.empty((n, k // g), dtype=torch.float16, device=w.device)
    with _dev(w):
        _lib.check(_lib.load().mp_w4_quantize_gptq_rtn(
            w.data_ptr(), _DT[w.dtype], n, k, g, iw.data_ptr(), packed.data_ptr(), scale.data_ptr(),
            _stream()), "mp_w4_quantize_gptq_rtn")
    return iw, packed, scale


def pack_int4(int_weight: torch.Tensor) -> torch.Tensor:
    """``pack_int4_for_vllm`` on the GPU (raises ValueError on out-of-range values)."""
    if int_weight.dim() != 2:
        raise ValueError(f"Expected 2D int_weight, got shape {tuple(int_weight.shape)}.")
    _need(int_weight, "int_weight", torch.int8, 2)
    n, k = int_weight.shape
    packed = torch.empty((n, (k + 7) // 8), dtype=torch.int32, device=int_weight.device)
    bad = torch.zeros(1, dtype=torch.int32, device=int_weight.device)
    with _dev(int_weight):
        _lib.check(_lib.load().mp_pack_int4(int_weight.data_ptr(), n, k, packed.data_ptr(), bad.data_ptr(),
                                            _stream()), "mp_pack_int4")
    if int(bad.item()) != 0:
        raise ValueError("int4 weights must be in signed range [-8, 7].")
    return packed


def unpack_int4(packed: torch.Tensor, k: int) -> torch.Tensor:
    _need(packed, "packed", torch.int32, 2)
    n = packed.shape[0]
    if packed.shape[1] != (k + 7) // 8:
        raise ValueError("packed width does not match k")
    out = torch.empty((n, k), dtype=torch.int8, device=packed.device)
    with _dev(packed):
        _lib.check(_lib.load().mp_unpack_int4(packed.data_ptr(), n, k, out.data_ptr(), _stream()), "mp_unpack_int4")
    return out


@torch.library.custom_op("mindpipe_amd::w4a16_gemm", mutates_args=())
def w4a16_gemm(x: torch.Tensor, w_packed: torch.Tensor, scales: torch.Tensor, zeros: Optional[torch.Tensor],
               group_size: int, bias: Optional[torch.Tensor]) -> torch.Tensor:
    """``Y = X . dequant(W)^T (+ bias)``; ``x`` fp16 or bf16 ``[..., K]`` (scales, zeros, bias and
    the output in the same dtype); ``w_packed`` int32 ``[N, K/8]``."""
    _need(x, "x", (torch.float16, torch.bfloat16))
    _need(w_packed, "w_packed", torch.int32, 2)
    _need(scales, "scales", x.dtype, 2)
    k = x.shape[-1]
    n = w_packed.shape[0]
    if w_packed.shape[1] * 8 != k:
        raise RuntimeError(f"w_packed {tuple(w_packed.shape)} does not match K={k}")
    if k % group_size or scales.shape != (n, k // group_size):
        raise RuntimeError(f"scales {tuple(scales.shape)} do not match N={n}, K={k}, g={group_size}")
    if zeros is not None:
        _need(zeros, "zeros", x.dtype, 2)
        if zeros.shape != scales.shape:
            raise RuntimeError("zeros must have the shape of scales")
    if bias is not None:
        _need(bias, "bias", x.dtype, 1)
        if bias.shape[0] != n:
            raise RuntimeError("bias must be [N]")
    x2 = x.reshape(-1, k)
    m = x2.shape[0]
    y = torch.empty((m, n), dtype=x.dtype, device=x.device)
    with _dev(x):
        _lib.check(_lib.load().mp_w4a16_gemm(
            x2.data_ptr(), m, k, w_packed.data_ptr(), n, scales.data_ptr(), _ptr(zeros), group_size,
            _ptr(bias), y.data_ptr(), _DT[x.dtype], _stream()), "mp_w4a16_gemm")
    return y.reshape(*x.shape[:-1], n)


@w4a16_gemm.register_fake
def _(x, w_packed, scales, zeros, group_size, bias):
    return x.new_empty((*x.shape[:-1], w_packed.shape[0]))


# ---------------------------------------------------------------- W8A8
@torch.library.custom_op("mindpipe_amd::quant_per_token_i8", mutates_args=())
def quant_per_token_i8(x: torch.Tensor, fake_rule: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-token dynamic int8 quant: ``(q int8 [..., K], scale [...])``.

    ``fake_rule=False``: fp32 scale ``absmax/127`` (``npu_dynamic_quant`` contract).
    ``fake_rule=True``: codes and scale (in ``x``'s dtype, fp16 or bf16) of
    ``quantize_activation_per_token_absmax``; ``q * scale`` is the reference's fake value
    (a bf16 row whose codes reach +128 is stored negated with a negated scale).
    """
    _need(x, "x", (torch.float16, torch.bfloat16, torch.float32))
    k = x.shape[-1]
    x2 = x.reshape(-1, k)
    m = x2.shape[0]
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    if fake_rule:
        if x.dtype not in (torch.float16, torch.bfloat16):
            raise RuntimeError("the fake rule takes fp16 or bf16 activations")
        s = torch.empty((m,), dtype=x.dtype, device=x.device)
    else:
        s = torch.empty((m,), dtype=torch.float32, device=x.device)
    with _dev(x):
        _lib.check(_lib.load().mp_quant_per_token_i8(
            x2.data_ptr(), m, k, _DT[x.dtype], q.data_ptr(), s.data_ptr(),
            MP_SCALE_FAKE if fake_rule else MP_SCALE_FP32, _stream()), "mp_quant_per_token_i8")
    return q.reshape(x.shape), s.reshape(x.shape[:-1])


@quant_per_token_i8.register_fake
def _(x, fake_rule=False):
    return (torch.empty_like(x, dtype=torch.int8),
            x.new_empty(x.shape[:-1], dtype=x.dtype if fake_rule else torch.float32))


def add_rms_norm_quant(x: torch.Tensor, residual: Optional[torch.Tensor], weight: torch.Tensor, eps: float,
                       quant: bool = True, out: bool = False, inplace: bool = False):
    """Fused residual add + RMSNorm + per-token dynamic int8 quant.

    Returns ``(y, q, scale, residual_sum)``: ``y`` the normalised activations in
    ``x.dtype`` (``None`` unless ``out`` or not ``quant``), ``q``/``scale`` the
    int8 codes and fp32 per-token scale of ``y`` (``None`` unless ``quant``) and
    ``residual_sum = x + residual`` in ``x.dtype`` (``None`` without a residual).
    ``inplace=True`` writes the sum into ``residual`` and ``y`` into ``x``
    (the in-place contract of vLLM's fused add-RMSNorm).
    """
    _need(x, "x", (torch.float16, torch.bfloat16))
    _need(weight, "weight", x.dtype, 1)
    h = x.shape[-1]
    if weight.shape[0] != h:
        raise RuntimeError(f"weight {tuple(weight.shape)} does not match H={h}")
    if residual is not None:
        _need(residual, "residual", x.dtype)
        if residual.shape != x.shape:
            raise RuntimeError("residual must have the shape of x")
    x2 = x.reshape(-1, h)
    m = x2.shape[0]
    want_y = out or not quant
    if inplace:
        y = x if want_y else None
        rsum = residual
    else:
        y = torch.empty_like(x) if want_y else None
        rsum = torch.empty_like(x) if residual is not None else None
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device) if quant else None
    s = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device) if quant else None
    with _dev(x):
        _lib.check(_lib.load().mp_add_rms_norm_quant(
            x2.data_ptr(), _ptr(residual), weight.data_ptr(), float(eps), m, h, _DT[x.dtype], _ptr(rsum),
            _ptr(y), _ptr(q), _ptr(s), _stream()), "mp_add_rms_norm_quant")
    return y, q, s, rsum


# Functional custom ops over the fused norm (fixed output schemas, fake implementations), the form
# torch.compile and graph capture take: the registration pattern of the reference's
# torch.ops.vllm.* ops (vllm.patch:171-228,291-306).
@torch.library.custom_op("mindpipe_amd::add_rms_norm_dynamic_quant", mutates_args=())
def add_rms_norm_dynamic_quant(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                               eps: float) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``(int8 codes, fp32 per-token scale, x + residual)`` of RMSNorm(x + residual) * weight
    (``npu_add_rms_norm_dynamic_quant``, ``vllm_ascend.patch:740-792``)."""
    _, q, sc, rsum = add_rms_norm_quant(x, residual, weight, eps, quant=True, out=False)
    return q, sc, rsum


@add_rms_norm_dynamic_quant.register_fake
def _(x, residual, weight, eps):
    return (torch.empty(x.shape, dtype=torch.int8, device=x.device),
            torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device), torch.empty_like(x))


@torch.library.custom_op("mindpipe_amd::rms_norm_dynamic_quant", mutates_args=())
def rms_norm_dynamic_quant(x: torch.Tensor, weight: torch.Tensor, eps: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """``(int8 codes, fp32 per-token scale)`` of RMSNorm(x) * weight (the first layer, no residual)."""
    _, q, sc, _ = add_rms_norm_quant(x, None, weight, eps, quant=True, out=False)
    return q, sc


@rms_norm_dynamic_quant.register_fake
def _(x, weight, eps):
    return (torch.empty(x.shape, dtype=torch.int8, device=x.device),
            torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device))


@torch.library.custom_op("mindpipe_amd::add_rms_norm", mutates_args=())
def add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                 eps: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """``(RMSNorm(x + residual) * weight, x + residual)`` in x's dtype (``npu_add_rms_norm``)."""
    y, _, _, rsum = add_rms_norm_quant(x, residual, weight, eps, quant=False)
    return y, rsum


@add_rms_norm.register_fake
def _(x, residual, weight, eps):
    return torch.empty_like(x), torch.empty_like(x)


def w8_quantize_per_channel(w: torch.Tensor, rule: str = "export"):
    """Per-output-channel int8 weight quant.

    ``rule="export"``: fp32 rule of the Ascend W8A8 export (clamp 1e-8).
    ``rule="fake"``: the rule of ``quantize_weight_per_channel_absmax`` in ``w``'s dtype
    (fp16 / bf16; a bf16 row whose codes reach +128 is stored negated with a negated scale).
    Returns ``(q int8 [N,K], scale_f32 [N], scale_src [N] in w.dtype)``.
    """
    _need(w, "w", (torch.float16, torch.bfloat16), 2)
    n, k = w.shape
    q = torch.empty((n, k), dtype=torch.int8, device=w.device)
    s32 = torch.empty((n,), dtype=torch.float32, device=w.device)
    ssrc = torch.empty((n,), dtype=w.dtype, device=w.device)
    bad = torch.zeros(1, dtype=torch.int32, device=w.device)
    r = MP_SCALE_FP32 if rule == "export" else MP_SCALE_FAKE
    if rule not in ("export", "fake"):
        raise ValueError(f"unknown rule {rule!r}")
    with _dev(w):
        _lib.check(_lib.load().mp_w8_quantize_per_channel(
            w.data_ptr(), n, k, _DT[w.dtype], q.data_ptr(), s32.data_ptr(), ssrc.data_ptr(), r, bad.data_ptr(),
            _stream()), "mp_w8_quantize_per_channel")
    if rule == "export" and int(bad.item()) != 0:
        raise ValueError("the weight holds non-finite values; the export quantizer needs finite weights")
    return q, s32, ssrc


@torch.library.custom_op("mindpipe_amd::w8a8_gemm", mutates_args=())
def w8a8_gemm(qx: torch.Tensor, s_tok: torch.Tensor, w: torch.Tensor, s_ch: torch.Tensor,
              bias: Optional[torch.Tensor], out_dtype: torch.dtype) -> torch.Tensor:
    """``((Qx . Qw^T) * s_tok) * s_ch (+ bias)`` -> ``out_dtype``; ``qx`` int8 ``[..., K]``, ``w`` int8 ``[N, K]``."""
    _need(qx, "qx", torch.int8)
    _need(w, "w", torch.int8, 2)
    _need(s_tok, "s_tok", torch.float32)
    _need(s_ch, "s_ch", torch.float32, 1)
    k = qx.shape[-1]
    n = w.shape[0]
    if w.shape[1] != k:
        raise RuntimeError(f"weight {tuple(w.shape)} does not match K={k}")
    q2 = qx.reshape(-1, k)
    m = q2.shape[0]
    if s_tok.numel() != m or s_ch.numel() != n:
        raise RuntimeError("scale sizes do not match M / N")
    if bias is not None:
        _need(bias, "bias", (torch.float16, torch.bfloat16, torch.float32), 1)
    y = torch.empty((m, n), dtype=out_dtype, device=qx.device)
    with _dev(qx):
        _lib.check(_lib.load().mp_w8a8_gemm(
            q2.data_ptr(), s_tok.data_ptr(), w.data_ptr(), s_ch.data_ptr(), _ptr(bias),
            _DT[bias.dtype] if bias is not None else MP_F16, y.data_ptr(), _DT[out_dtype], m, n, k, _stream()),
            "mp_w8a8_gemm")
    return y.reshape(*qx.shape[:-1], n)


@w8a8_gemm.register_fake
def _(qx, s_tok, w, s_ch, bias, out_dtype):
    return qx.new_empty((*qx.shape[:-1], w.shape[0]), dtype=out_dtype)


@torch.library.custom_op("mindpipe_amd::w8a8_gemm_fake", mutates_args=())
def w8a8_gemm_fake(qx: torch.Tensor, s_tok: torch.Tensor, w: torch.Tensor, s_ch: torch.Tensor,
                   bias: Optional[torch.Tensor], act_dtype: torch.dtype) -> torch.Tensor:
    """``F.linear(r(qx * s_tok), r(w * s_ch), bias)`` in ``act_dtype`` (fp16 / bf16): the fake
    path of ``SmoothQuantLinear.forward`` (``fake_quant.py:85-88``) on the fake rule's codes,
    every operand element rounded as the reference's fake-quant tensors are."""
    _need(qx, "qx", torch.int8)
    _need(w, "w", torch.int8, 2)
    _need(s_tok, "s_tok", torch.float32)
    _need(s_ch, "s_ch", torch.float32, 1)
    if act_dtype not in (torch.float16, torch.bfloat16):
        raise RuntimeError("the fake path runs in fp16 or bf16")
    k = qx.shape[-1]
    n = w.shape[0]
    if w.shape[1] != k:
        raise RuntimeError(f"weight {tuple(w.shape)} does not match K={k}")
    q2 = qx.reshape(-1, k)
    m = q2.shape[0]
    if s_tok.numel() != m or s_ch.numel() != n:
        raise RuntimeError("scale sizes do not match M / N")
    if bias is not None:
        _need(bias, "bias", act_dtype, 1)
    y = torch.empty((m, n), dtype=act_dtype, device=qx.device)
    with _dev(qx):
        _lib.check(_lib.load().mp_w8a8_gemm_fake(
            q2.data_ptr(), s_tok.data_ptr(), w.data_ptr(), s_ch.data_ptr(), _ptr(bias), _DT[act_dtype],
            y.data_ptr(), m, n, k, _stream()), "mp_w8a8_gemm_fake")
    return y.reshape(*qx.shape[:-1], n)


@w8a8_gemm_fake.register_fake
def _(qx, s_tok, w, s_ch, bias, act_dtype):
    return qx.new_empty((*qx.shape[:-1], w.shape[0]), dtype=act_dtype)


# ---------------------------------------------------------------- MoE
_RULES = {"runtime": MP_SCALE_FP32, "fake": MP_SCALE_FAKE}


def fake_quant_rows(x: torch.Tensor, n_bits: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-row fake quant at ``n_bits`` = 2..7 (``quantize_*_absmax`` with ``n_bits < 8``) in the
    arithmetic of ``x``'s dtype (fp16 / bf16): ``(int8 codes [.., K], fp32 scale [..])``; the fake
    value is ``r(q * s)``."""
    _need(x, "x", (torch.float16, torch.bfloat16))
    k = x.shape[-1]
    x2 = x.reshape(-1, k)
    q = torch.empty(x2.shape, dtype=torch.int8, device=x.device)
    s = torch.empty((x2.shape[0],), dtype=torch.float32, device=x.device)
    with _dev(x):
        _lib.check(_lib.load().mp_fake_quant_rows(x2.data_ptr(), _DT[x.dtype], x2.shape[0], k, int(n_bits),
                                                  q.data_ptr(), s.data_ptr(), _stream()), "mp_fake_quant_rows")
    return q.reshape(x.shape), s.reshape(x.shape[:-1])


def dq_linear(a: torch.Tensor, a_scale: Optional[torch.Tensor], b: torch.Tensor, b_scale: Optional[torch.Tensor],
              bias: Optional[torch.Tensor], dtype: torch.dtype) -> torch.Tensor:
    """``F.linear(A, B, bias)`` in ``dtype`` (fp16 / bf16) where A is int8 codes with a per-row fp32
    scale (the fake value ``r(q * s)``) or, with ``a_scale`` None, plain values in ``dtype``; B
    likewise ([N, K]).  fp32 accumulation, one rounding: the fake-quant linear at any operand widths."""
    if dtype not in (torch.float16, torch.bfloat16):
        raise RuntimeError("the fake-quant linear runs in fp16 or bf16")
    k = a.shape[-1]
    a2 = a.reshape(-1, k)
    m = a2.shape[0]
    _need(a2, "a", torch.int8 if a_scale is not None else dtype, 2)
    _need(b, "b", torch.int8 if b_scale is not None else dtype, 2)
    n = b.shape[0]
    if b.shape[1] != k:
        raise RuntimeError(f"b {tuple(b.shape)} does not match K={k}")
    if a_scale is not None:
        _need(a_scale, "a_scale", torch.float32)
        if a_scale.numel() != m:
            raise RuntimeError("a_scale does not match the rows of a")
    if b_scale is not None:
        _need(b_scale, "b_scale", torch.float32, 1)
        if b_scale.numel() != n:
            raise RuntimeError("b_scale does not match the rows of b")
    if bias is not None:
        _need(bias, "bias", dtype, 1)
    y = torch.empty((m, n), dtype=dtype, device=a.device)
    with _dev(a):
        _lib.check(_lib.load().mp_dq_linear(a2.data_ptr(), _ptr(a_scale), b.data_ptr(), _ptr(b_scale), _ptr(bias),
                                            _DT[dtype], y.data_ptr(), m, n, k, _stream()), "mp_dq_linear")
    return y.reshape(*a.shape[:-1], n)


@torch.library.custom_op("mindpipe_amd::w8a8_gemm_quant_out", mutates_args=())
def w8a8_gemm_quant_out(qx: torch.Tensor, s_tok: torch.Tensor, w: torch.Tensor, s_ch: torch.Tensor,
                        bias: Optional[torch.Tensor], out_dtype: torch.dtype,
                        fake_rule: bool = False) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``(y, q, s)``: the W8A8 linear's output ``y [M, N]`` in ``out_dtype`` (fp16 / bf16) and its
    per-token int8 codes and scale, from the GEMM epilogue's row abs-max (``quantize_output``,
    ``fake_quant.py:77-82``).  ``fake_rule``: the reference's fake rule in ``out_dtype`` (else the
    fp32 runtime rule)."""
    _need(qx, "qx", torch.int8, 2)
    _need(w, "w", torch.int8, 2)
    _need(s_tok, "s_tok", torch.float32, 1)
    _need(s_ch, "s_ch", torch.float32, 1)
    if out_dtype not in (torch.float16, torch.bfloat16):
        raise RuntimeError(f"w8a8_gemm_quant_out writes fp16 or bf16, got {out_dtype}")
    m, k = qx.shape
    n = w.shape[0]
    if w.shape[1] != k or s_tok.numel() != m or s_ch.numel() != n:
        raise RuntimeError("w8a8_gemm_quant_out: operand shapes disagree")
    if bias is not None:
        _need(bias, "bias", (torch.float16, torch.bfloat16, torch.float32), 1)
    y = torch.empty((m, n), dtype=out_dtype, device=qx.device)
    q = torch.empty((m, n), dtype=torch.int8, device=qx.device)
    sc = torch.empty((m,), dtype=torch.float32, device=qx.device)
    lib = _lib.load()
    ws = torch.empty(max(16, int(lib.mp_w8a8_gemm_quant_out_workspace_bytes(m, n))), dtype=torch.uint8,
                     device=qx.device)
    with _dev(qx):
        _lib.check(lib.mp_w8a8_gemm_quant_out(
            qx.data_ptr(), s_tok.data_ptr(), w.data_ptr(), s_ch.data_ptr(), _ptr(bias),
            _DT[bias.dtype] if bias is not None else 0, m, n, k, _DT[out_dtype],
            MP_SCALE_FAKE if fake_rule else MP_SCALE_FP32, y.data_ptr(), q.data_ptr(), sc.data_ptr(), ws.data_ptr(),
            ws.numel(), _stream()), "mp_w8a8_gemm_quant_out")
    return y, q, sc


@w8a8_gemm_quant_out.register_fake
def _(qx, s_tok, w, s_ch, bias, out_dtype, fake_rule=False):
    m, n = qx.shape[0], w.shape[0]
    return (torch.empty((m, n), dtype=out_dtype, device=qx.device),
            torch.empty((m, n), dtype=torch.int8, device=qx.device),
            torch.empty((m,), dtype=torch.float32, device=qx.device))


def _rule(rule: str) -> int:
    if rule not in _RULES:
        raise ValueError(f"unknown scale rule {rule!r} (expected 'runtime' or 'fake')")
    return _RULES[rule]


def moe_permute_quant(x: torch.Tensor, topk_ids: torch.Tensor, n_experts: int, rule: str = "runtime",
                      x_scale: Optional[torch.Tensor] = None):
    """Routing + per-token quant: ``(routed int8 [T*k,H], routed_scale f32, row_of_slot int32 [T*k],
    group_offsets int64 [E+1])``.  Rows of ``routed`` past ``group_offsets[-1]`` are unused.

    ``rule="runtime"``: fp32 scale ``absmax/127``; ``rule="fake"``: the reference module's
    ``act_quant`` in ``x``'s dtype (fp16 / bf16).  With ``x_scale`` (fp32 ``[T]``), ``x`` is
    already int8 (the runtime's ``pertoken_scale`` input) and is routed without re-quantizing."""
    if x_scale is not None:
        _need(x, "x", torch.int8, 2)
        _need(x_scale, "x_scale", torch.float32)
        if x_scale.numel() != x.shape[0]:
            raise RuntimeError("x_scale must hold one scale per token")
        x_dt = MP_I8
    else:
        _need(x, "x", (torch.float16, torch.bfloat16, torch.float32), 2)
        x_dt = _DT[x.dtype]
    _need(topk_ids, "topk_ids", torch.int32, 2)
    t, h = x.shape
    top_k = topk_ids.shape[1]
    if topk_ids.shape[0] != t:
        raise RuntimeError("topk_ids must be [T, top_k]")
    lib = _lib.load()
    rows = t * top_k
    routed = torch.empty((rows, h), dtype=torch.int8, device=x.device)
    rscale = torch.empty((rows,), dtype=torch.float32, device=x.device)
    row_of_slot = torch.empty((rows,), dtype=torch.int32, device=x.device)
    offsets = torch.empty((n_experts + 1,), dtype=torch.int64, device=x.device)
    wsb = lib.mp_moe_route_workspace_bytes(t, h, n_experts)
    ws = torch.zeros((wsb,), dtype=torch.uint8, device=x.device)
    with _dev(x):
        _lib.check(lib.mp_moe_permute_quant(
            x.data_ptr(), x_dt, _ptr(x_scale), t, h, topk_ids.data_ptr(), top_k, n_experts, _rule(rule),
            routed.data_ptr(), rscale.data_ptr(), row_of_slot.data_ptr(), offsets.data_ptr(), ws.data_ptr(), wsb,
            _stream()), "mp_moe_permute_quant")
    return routed, rscale, row_of_slot, offsets


@torch.library.custom_op("mindpipe_amd::i8_gemm_swiglu_requant", mutates_args=())
def moe_gmm1_swiglu_quant(routed: torch.Tensor, rscale: torch.Tensor, w13: torch.Tensor, s13: torch.Tensor,
                          offsets: torch.Tensor, inter: int, rule: str = "runtime",
                          act_dtype: torch.dtype = torch.float16) -> Tuple[torch.Tensor, torch.Tensor]:
    """GMM1 + SwiGLU + requant over expert groups: ``(q int8 [R, I], s f32 [R])``.  The
    counterpart of the reference bridge op ``mindpipe_qwen2_grouped_swiglu_loop_out``
    (``aclnn_grouped_swiglu_out_bridge.cpp:157-273``) with no 10240-column limit.
    ``rule="fake"`` rounds gate, up, silu(gate) and h in ``act_dtype`` and requantizes with the
    fake rule (the reference module's forward); ``"runtime"`` keeps fp32."""
    _need(routed, "routed", torch.int8, 2)
    _need(rscale, "routed_scale", torch.float32, 1)
    _need(w13, "w13", torch.int8, 3)
    _need(s13, "s13", torch.float32, 2)
    _need(offsets, "group_offsets", torch.int64, 1)
    rows, h = routed.shape
    e = w13.shape[0]
    if w13.shape[1] != 2 * inter or w13.shape[2] != h or s13.shape != (e, 2 * inter):
        raise RuntimeError("w13 must be [E, 2I, H] with s13 [E, 2I]")
    if offsets.numel() != e + 1 or rscale.numel() != rows:
        raise RuntimeError("group_offsets must be [E+1] and routed_scale [R]")
    lib = _lib.load()
    q = torch.empty((rows, inter), dtype=torch.int8, device=routed.device)
    s = torch.empty((rows,), dtype=torch.float32, device=routed.device)
    wsb = lib.mp_moe_gmm1_workspace_bytes(rows, inter)
    ws = torch.empty((wsb,), dtype=torch.uint8, device=routed.device)
    with _dev(routed):
        _lib.check(lib.mp_i8_gemm_swiglu_requant(
            routed.data_ptr(), rscale.data_ptr(), w13.data_ptr(), s13.data_ptr(), offsets.data_ptr(), e, rows, h,
            inter, _rule(rule), _DT[act_dtype], q.data_ptr(), s.data_ptr(), ws.data_ptr(), wsb, _stream()),
            "mp_i8_gemm_swiglu_requant")
    return q, s


@moe_gmm1_swiglu_quant.register_fake
def _(routed, rscale, w13, s13, offsets, inter, rule="runtime", act_dtype=torch.float16):
    return (routed.new_empty((routed.shape[0], inter), dtype=torch.int8),
            routed.new_empty((routed.shape[0],), dtype=torch.float32))


def moe_gmm2(q, s, w2, s2, offsets, out_dtype=torch.float32, rule: str = "runtime",
             act_dtype: torch.dtype = torch.float16):
    """Grouped GEMM2 ``[R, N]``: the int8 product with the per-token x per-row epilogue
    (``rule="runtime"``), or ``F.linear`` of the fake-quant tensors in ``act_dtype``
    (``rule="fake"``)."""
    _need(q, "q", torch.int8, 2)
    _need(s, "s", torch.float32, 1)
    _need(w2, "w2", torch.int8, 3)
    _need(s2, "s2", torch.float32, 2)
    _need(offsets, "group_offsets", torch.int64, 1)
    rows, k = q.shape
    e, n, k2 = w2.shape
    if k2 != k or s2.shape != (e, n) or offsets.numel() != e + 1 or s.numel() != rows:
        raise RuntimeError("w2 must be [E, H, I] with s2 [E, H], group_offsets [E+1], s [R]")
    y = torch.empty((rows, n), dtype=out_dtype, device=q.device)
    with _dev(q):
        _lib.check(_lib.load().mp_w8a8_grouped_gemm(
            q.data_ptr(), s.data_ptr(), w2.data_ptr(), s2.data_ptr(), offsets.data_ptr(), e, rows, n, k,
            _rule(rule), _DT[act_dtype], y.data_ptr(), _DT[out_dtype], _stream()), "mp_w8a8_grouped_gemm")
    return y


def moe_unpermute_combine(y, row_of_slot, topk_w, out_dtype=torch.float16, rule: str = "runtime"):
    """``rule="runtime"``: fp32 weighted sum in slot order, one rounding; ``rule="fake"``: the
    reference's ``index_add_`` in ``out_dtype`` over ascending experts."""
    _need(y, "y", torch.float32, 2)
    _need(row_of_slot, "row_of_slot", torch.int32, 1)
    _need(topk_w, "topk_weights", torch.float32, 2)
    t, top_k = topk_w.shape
    h = y.shape[1]
    if row_of_slot.numel() != t * top_k:
        raise RuntimeError("row_of_slot must hold T * top_k entries")
    out = torch.empty((t, h), dtype=out_dtype, device=y.device)
    with _dev(y):
        _lib.check(_lib.load().mp_moe_unpermute_combine(
            y.data_ptr(), row_of_slot.data_ptr(), topk_w.data_ptr(), t, top_k, h, _rule(rule), out.data_ptr(),
            _DT[out_dtype], _stream()), "mp_moe_unpermute_combine")
    return out


@torch.library.custom_op("mindpipe_amd::moe_w8a8_forward", mutates_args=())
def moe_w8a8_forward(x: torch.Tensor, topk_ids: torch.Tensor, topk_w: torch.Tensor, w13: torch.Tensor,
                     s13: torch.Tensor, w2: torch.Tensor, s2: torch.Tensor, out_dtype: Optional[torch.dtype] = None,
                     rule: str = "runtime", x_scale: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Whole W8A8 MoE chain (routing quant -> GMM1+SwiGLU+requant -> GMM2 -> combine) on the
    kernel layout ``w13 [E, 2I, H]``, ``w2 [E, H, I]`` with fp32 per-row scales.

    ``rule="fake"`` reproduces ``SmoothQuantPackedMoeExperts.forward`` (``fake_quant.py:166-191``)
    in ``x``'s dtype; ``rule="runtime"`` is the fp32-scale chain of ``_run_expert_tile``
    (``vllm_ascend.patch:2356-2423``).  ``x_scale`` marks ``x`` as pre-quantized int8."""
    e = w13.shape[0]
    inter = w2.shape[2]
    if out_dtype is None:
        out_dtype = x.dtype if x_scale is None else torch.float16
    act_dtype = x.dtype if x_scale is None else out_dtype
    if rule == "fake" and act_dtype not in (torch.float16, torch.bfloat16):
        raise RuntimeError("the fake rule runs in fp16 or bf16")
    routed, rscale, row_of_slot, offsets = moe_permute_quant(x, topk_ids.to(torch.int32).contiguous(), e, rule,
                                                             x_scale)
    q, s = moe_gmm1_swiglu_quant(routed, rscale, w13, s13, offsets, inter, rule, act_dtype)
    y = moe_gmm2(q, s, w2, s2, offsets, torch.float32, rule, act_dtype)
    return moe_unpermute_combine(y, row_of_slot, topk_w.to(torch.float32).contiguous(), out_dtype, rule)


@moe_w8a8_forward.register_fake
def _(x, topk_ids, topk_w, w13, s13, w2, s2, out_dtype=None, rule="runtime", x_scale=None):
    if out_dtype is None:
        out_dtype = x.dtype if x_scale is None else torch.float16
    return x.new_empty((x.shape[0], w2.shape[1]), dtype=out_dtype)


@torch.library.custom_op("mindpipe_amd::dense_mlp_w8a8", mutates_args=())
def dense_mlp_w8a8(qx: torch.Tensor, sx: torch.Tensor, offsets: torch.Tensor, w13_chunks: List[torch.Tensor],
                   s13_chunks: List[torch.Tensor], w2_chunks: torch.Tensor, s2: torch.Tensor, chunk_size: int,
                   out_dtype: torch.dtype) -> torch.Tensor:
    """The chunked W8A8 MLP chain (``vllm.patch:883-937``; one chunk ``:1003-1037``): per chunk, GEMM1
    + SwiGLU + requant over one group of all T tokens (``offsets = [0, T]``), then the int8 down GEMM
    on the chunk's columns; one chunk writes ``out_dtype`` directly, several are summed in fp32 and
    rounded once.  ``w13_chunks[c] [1, 2cs, H]`` / ``s13_chunks[c] [1, 2cs]`` fp32, ``w2_chunks
    [chunks, H, cs]``, ``s2 [H]`` fp32."""
    chunks = len(w13_chunks)
    if chunks == 0 or len(s13_chunks) != chunks or w2_chunks.shape[0] != chunks:
        raise ValueError("dense_mlp_w8a8: chunk lists disagree")
    out = None
    for c in range(chunks):
        qh, sh = moe_gmm1_swiglu_quant(qx, sx, w13_chunks[c], s13_chunks[c], offsets, chunk_size)
        if chunks == 1:
            return w8a8_gemm(qh, sh, w2_chunks[0], s2, None, out_dtype)
        y = w8a8_gemm(qh, sh, w2_chunks[c], s2, None, torch.float32)
        out = y if out is None else out + y
    return out.to(out_dtype)


@dense_mlp_w8a8.register_fake
def _(qx, sx, offsets, w13_chunks, s13_chunks, w2_chunks, s2, chunk_size, out_dtype):
    return torch.empty((qx.shape[0], w2_chunks.shape[1]), dtype=out_dtype, device=qx.device)


def group_offsets_from_list(group_list: torch.Tensor, group_list_type: int) -> torch.Tensor:
    """``group_offsets [E+1]`` (leading 0) from the runtime's ``group_list [E]``: cumulative
    endpoints (type 0) or raw counts (type 1) (``vllm_ascend.patch:2015-2031``)."""
    if group_list_type not in (0, 1):
        raise ValueError(f"group_list_type must be 0 (cumulative) or 1 (counts), got {group_list_type}")
    gl = group_list.to(torch.int64).reshape(-1)
    ends = gl if group_list_type == 0 else torch.cumsum(gl, 0)
    return torch.cat([ends.new_zeros(1), ends]).contiguous()


# ---------------------------------------------------------------- decode-step harness kernels
def w4a16_gemm_swiglu(x: torch.Tensor, w_packed: torch.Tensor, scales: torch.Tensor, zeros: Optional[torch.Tensor],
                      group_size: int, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``silu(G) * U`` with ``[G | U] = X . dequant(W)^T (+ bias)`` for the fused gate/up weight
    ``w_packed [2I, K/8]`` (gate rows first): ``[..., I]`` in ``x``'s dtype (fp16 or bf16), rounded as
    ``silu_mul`` of the ``w4a16_gemm`` output.  One launch (group 128, K % 256 == 0, M * K and M * I
    below 2^30); otherwise the two launches."""
    k = x.shape[-1]
    n2 = w_packed.shape[0]
    x2 = x.reshape(-1, k)
    m = x2.shape[0]
    if group_size != 128 or k % 256 or n2 % 2 or m * k >= (1 << 30) or m * (n2 // 2) >= (1 << 30):
        return silu_mul(w4a16_gemm(x2, w_packed, scales, zeros, group_size, bias)).reshape(*x.shape[:-1], n2 // 2)
    _need(x, "x", (torch.float16, torch.bfloat16))
    _need(w_packed, "w_packed", torch.int32, 2)
    _need(scales, "scales", x.dtype, 2)
    if w_packed.shape[1] * 8 != k or scales.shape != (n2, k // group_size):
        raise RuntimeError(f"w_packed {tuple(w_packed.shape)} / scales {tuple(scales.shape)} do not match K={k}")
    if zeros is not None and (zeros.shape != scales.shape or zeros.dtype != x.dtype):
        raise RuntimeError("zeros must have the shape and dtype of scales")
    if bias is not None and bias.shape != (n2,):
        raise RuntimeError("bias must be [2I]")
    if bias is not None and bias.dtype != x.dtype:
        raise RuntimeError("bias must have the activation dtype")
    act = torch.empty((m, n2 // 2), dtype=x.dtype, device=x.device)
    with _dev(x):
        _lib.check(_lib.load().mp_w4a16_gemm_swiglu(
            x2.data_ptr(), m, k, w_packed.data_ptr(), n2, scales.data_ptr(), _ptr(zeros), group_size,
            _ptr(bias), act.data_ptr(), _DT[x.dtype], _stream()), "mp_w4a16_gemm_swiglu")
    return act.reshape(*x.shape[:-1], n2 // 2)


def w4a16_gemv_add_rms_norm(x: torch.Tensor, residual: Optional[torch.Tensor], norm_weight: torch.Tensor,
                            eps: float, w_packed: torch.Tensor, scales: torch.Tensor, zeros: Optional[torch.Tensor],
                            group_size: int, bias: Optional[torch.Tensor] = None, swiglu: bool = False):
    """One fp16 row ``x [1, K]``: ``(y, residual_sum)`` with ``residual_sum = x + residual``
    (``None`` without a residual) and ``y`` the W4A16 linear (``swiglu``: the SiLU-up product
    of the fused gate/up weight) of ``RMSNorm(x + residual) * norm_weight``, in one launch.
    The same bits as ``add_rms_norm_quant(..., quant=False)`` followed by ``w4a16_gemm`` /
    ``w4a16_gemm_swiglu``.  K in {2048, 4096, 8192}, group 128."""
    _need(x, "x", torch.float16)
    _need(norm_weight, "norm_weight", torch.float16, 1)
    _need(w_packed, "w_packed", torch.int32, 2)
    _need(scales, "scales", torch.float16, 2)
    k = x.shape[-1]
    if x.numel() != k:
        raise RuntimeError(f"x must hold one row, got {tuple(x.shape)}")
    n = w_packed.shape[0]
    if w_packed.shape[1] * 8 != k or norm_weight.shape[0] != k:
        raise RuntimeError(f"w_packed {tuple(w_packed.shape)} / norm_weight do not match K={k}")
    if scales.shape != (n, k // group_size) or (zeros is not None and zeros.shape != scales.shape):
        raise RuntimeError(f"scales / zeros do not match N={n}, K={k}, g={group_size}")
    if residual is not None:
        _need(residual, "residual", torch.float16)
        if residual.shape != x.shape:
            raise RuntimeError("residual must have the shape of x")
    if bias is not None and bias.shape != (n,):
        raise RuntimeError("bias must be [N]")
    y = torch.empty((*x.shape[:-1], n // 2 if swiglu else n), dtype=torch.float16, device=x.device)
    rsum = torch.empty_like(x) if residual is not None else None
    with _dev(x):
        _lib.check(_lib.load().mp_w4a16_gemv_rmsnorm(
            x.data_ptr(), _ptr(residual), norm_weight.data_ptr(), float(eps), _ptr(rsum), k, w_packed.data_ptr(),
            n, scales.data_ptr(), _ptr(zeros), group_size, _ptr(bias), 1 if swiglu else 0, y.data_ptr(), MP_F16,
            _stream()), "mp_w4a16_gemv_rmsnorm")
    return y, rsum


def _decode_checks(b: int, nh: int, kvh: int, k_cache: torch.Tensor, v_cache: torch.Tensor, pos: torch.Tensor,
                   qkv: Optional[torch.Tensor] = None, q: Optional[torch.Tensor] = None,
                   cos_t: Optional[torch.Tensor] = None, sin_t: Optional[torch.Tensor] = None,
                   out: Optional[torch.Tensor] = None) -> None:
    """Shapes the decode kernels assume (the C ABI sees pointers only, so a wrong extent would become
    an out-of-bounds access instead of an error): head dim 128, caches ``[B, kvh, T, 128]`` fp16,
    RoPE tables ``[>= T, 64]`` fp16, ``pos`` one int64, outputs ``[B, nh, 128]`` fp16."""
    if nh <= 0 or kvh <= 0 or nh % kvh:
        raise RuntimeError(f"heads {nh} must be a positive multiple of kv heads {kvh}")
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        _need(c, name, torch.float16, 4)
        if c.shape[0] != b or c.shape[1] != kvh or c.shape[3] != 128:
            raise RuntimeError(f"{name} must be [{b}, {kvh}, T, 128], got {tuple(c.shape)}")
    if v_cache.shape != k_cache.shape:
        raise RuntimeError("k_cache and v_cache must have one shape")
    _need(pos, "pos", torch.int64)
    if pos.numel() != 1:
        raise RuntimeError("pos must hold one position")
    if qkv is not None:
        _need(qkv, "qkv", torch.float16, 2)
        if qkv.shape != (b, (nh + 2 * kvh) * 128):
            raise RuntimeError(f"qkv must be [{b}, {(nh + 2 * kvh) * 128}], got {tuple(qkv.shape)}")
    if q is not None:
        _need(q, "q", torch.float16, 3)
        if q.shape != (b, nh, 128):
            raise RuntimeError(f"q must be [{b}, {nh}, 128], got {tuple(q.shape)}")
    for name, t in (("cos_t", cos_t), ("sin_t", sin_t)):
        if t is not None:
            _need(t, name, torch.float16, 2)
            if t.shape[0] < k_cache.shape[2] or t.shape[1] != 64:
                raise RuntimeError(f"{name} must be [>= {k_cache.shape[2]}, 64], got {tuple(t.shape)}")
    if out is not None:
        _need(out, "out", torch.float16, 3)
        if out.shape != (b, nh, 128):
            raise RuntimeError(f"out must be [{b}, {nh}, 128], got {tuple(out.shape)}")


def decode_rope_append(qkv: torch.Tensor, nh: int, kvh: int, cos_t: torch.Tensor, sin_t: torch.Tensor,
                       pos: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                       q_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """RoPE on q/k of ``qkv [B, (nh+2kvh)*128]`` and append k/v at ``pos`` (int64 device scalar)
    into ``k_cache``/``v_cache [B, kvh, T, 128]``; returns rotated ``q [B, nh, 128]``."""
    b = qkv.shape[0]
    _decode_checks(b, nh, kvh, k_cache, v_cache, pos, qkv=qkv, cos_t=cos_t, sin_t=sin_t, out=q_out)
    cap = k_cache.shape[2]
    if q_out is None:
        q_out = torch.empty((b, nh, 128), dtype=torch.float16, device=qkv.device)
    with _dev(qkv):
        _lib.check(_lib.load().mp_decode_rope_append(
            qkv.data_ptr(), b, nh, kvh, 128, cos_t.data_ptr(), sin_t.data_ptr(), pos.data_ptr(), cap,
            q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), _stream()), "mp_decode_rope_append")
    return q_out


def prefill_rope_split(qkv: torch.Tensor, batch: int, nh: int, kvh: int, cos_t: torch.Tensor, sin_t: torch.Tensor,
                       k_cache: torch.Tensor, v_cache: torch.Tensor) -> torch.Tensor:
    """Prefill of positions ``0 .. T-1``: ``qkv [B*T, (nh+2kvh)*128]`` fp16 (each sequence's token rows
    in order).  RoPE on the q / k heads (the fp16 ops of ``decode_rope_append``), the rotated keys and
    the values written into ``k_cache`` / ``v_cache [B, kvh, cap, 128]`` at positions ``0 .. T-1``;
    returns the rotated queries ``[B, nh, T, 128]``."""
    _need(qkv, "qkv", torch.float16, 2)
    _need(cos_t, "cos_t", torch.float16, 2)
    _need(sin_t, "sin_t", torch.float16, 2)
    if batch < 1:
        raise RuntimeError(f"batch must be >= 1, got {batch}")
    for name, c in (("cos_t", cos_t), ("sin_t", sin_t), ("k_cache", k_cache), ("v_cache", v_cache)):
        if c.device != qkv.device:
            raise RuntimeError(f"{name} is on {c.device}, qkv on {qkv.device}")
    if qkv.shape[0] % batch != 0 or qkv.shape[1] != (nh + 2 * kvh) * 128:
        raise RuntimeError(f"qkv must be [B*T, {(nh + 2 * kvh) * 128}], got {tuple(qkv.shape)}")
    t = qkv.shape[0] // batch
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        _need(c, name, torch.float16, 4)
        if c.shape[0] != batch or c.shape[1] != kvh or c.shape[3] != 128 or not c.is_contiguous():
            raise RuntimeError(f"{name} must be a contiguous [{batch}, {kvh}, cap, 128], got {tuple(c.shape)}")
    cap = k_cache.shape[2]
    if v_cache.shape[2] != cap or t > cap or cos_t.shape != (cap, 64) or sin_t.shape != (cap, 64):
        raise RuntimeError("cache capacity, cos / sin rows and T do not match")
    q = torch.empty((batch, nh, t, 128), dtype=torch.float16, device=qkv.device)
    with _dev(qkv):
        _lib.check(_lib.load().mp_prefill_rope_split(
            qkv.data_ptr(), batch, t, nh, kvh, 128, cos_t.data_ptr(), sin_t.data_ptr(), cap, q.data_ptr(),
            k_cache.data_ptr(), v_cache.data_ptr(), _stream()), "mp_prefill_rope_split")
    return q


def decode_attention_workspace(batch: int, nh: int, splits: int, device) -> torch.Tensor:
    """Workspace of the decode attention: the splits' partial outputs and statistics."""
    nbytes = _lib.load().mp_decode_attention_workspace_bytes(batch, nh, splits)
    return torch.empty((nbytes // 4,), dtype=torch.float32, device=device)


def decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, pos: torch.Tensor, splits: int,
                     scale: float, workspace: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Attention of ``q [B, nh, 128]`` over cache positions ``[0, pos]``: ``[B, nh, 128]`` fp16."""
    _need(q, "q", torch.float16, 3)
    b, nh, hd = q.shape
    _need(workspace, "workspace", torch.float32, 1)
    _decode_checks(b, nh, k_cache.shape[1] if k_cache.dim() == 4 else 1, k_cache, v_cache, pos, q=q, out=out)
    kvh, cap = k_cache.shape[1], k_cache.shape[2]
    if out is None:
        out = torch.empty_like(q)
    with _dev(q):
        _lib.check(_lib.load().mp_decode_attention(
            q.data_ptr(), b, nh, kvh, hd, k_cache.data_ptr(), v_cache.data_ptr(), pos.data_ptr(), cap, splits,
            float(scale), out.data_ptr(), workspace.data_ptr(), workspace.numel() * 4, _stream()),
            "mp_decode_attention")
    return out


def decode_rope_attention(qkv: torch.Tensor, nh: int, kvh: int, cos_t: torch.Tensor, sin_t: torch.Tensor,
                          pos: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, splits: int, scale: float,
                          workspace: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``decode_rope_append`` + ``decode_attention`` in one launch: RoPE on the q/k heads of
    ``qkv [B, (nh+2kvh)*128]``, k/v appended at ``pos``, attention over ``[0, pos]``;
    returns ``[B, nh, 128]`` fp16."""
    b = qkv.shape[0]
    _need(workspace, "workspace", torch.float32, 1)
    _decode_checks(b, nh, kvh, k_cache, v_cache, pos, qkv=qkv, cos_t=cos_t, sin_t=sin_t, out=out)
    cap = k_cache.shape[2]
    if out is None:
        out = torch.empty((b, nh, 128), dtype=torch.float16, device=qkv.device)
    with _dev(qkv):
        _lib.check(_lib.load().mp_decode_rope_attention(
            qkv.data_ptr(), b, nh, kvh, 128, cos_t.data_ptr(), sin_t.data_ptr(), pos.data_ptr(), cap,
            k_cache.data_ptr(), v_cache.data_ptr(), splits, float(scale), out.data_ptr(), workspace.data_ptr(),
            workspace.numel() * 4, _stream()), "mp_decode_rope_attention")
    return out


def argmax_rows(x: torch.Tensor) -> torch.Tensor:
    """``x.argmax(-1)`` of fp16 ``x [rows, n]`` (first index of the maximum; NaN counts as the
    maximum), int64 ``[rows]``: the decode step's greedy sampling in one launch."""
    _need(x, "x", torch.float16, 2)
    rows, n = x.shape
    out = torch.empty(rows, dtype=torch.int64, device=x.device)
    with _dev(x):
        _lib.check(_lib.load().mp_argmax_rows(x.data_ptr(), rows, n, out.data_ptr(), _stream()), "mp_argmax_rows")
    return out


def silu_mul(gate_up: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``round(round(silu(gate)) * up)`` of ``gate_up [B, 2I]`` (gate | up), fp16 or bf16 (every round
    to that dtype)."""
    _need(gate_up, "gate_up", (torch.float16, torch.bfloat16), 2)
    rows, two_i = gate_up.shape
    if out is None:
        out = torch.empty((rows, two_i // 2), dtype=gate_up.dtype, device=gate_up.device)
    with _dev(gate_up):
        _lib.check(_lib.load().mp_silu_mul(gate_up.data_ptr(), rows, two_i // 2, out.data_ptr(), _DT[gate_up.dtype],
                                           _stream()), "mp_silu_mul")
    return out


# ------------------------------------------------------------------ SmoothQuant smoothing
_DT3 = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def colmax_abs(x: torch.Tensor, colmax: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Per-column ``max |x|`` over the rows of ``x [..., K]`` (fp16 / bf16 / fp32) into the fp32
    vector ``colmax [K]``: a new one, or the given one updated in place with the running maximum."""
    if x.dtype not in _DT3:
        raise RuntimeError(f"colmax_abs takes fp16, bf16 or fp32, got {x.dtype}")
    if not x.is_cuda:
        raise RuntimeError("colmax_abs runs on the GPU only")
    k = x.shape[-1]
    x2 = x.reshape(-1, k)
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    acc = colmax is not None
    if colmax is None:
        colmax = torch.empty(k, dtype=torch.float32, device=x.device)
    _need(colmax, "colmax", torch.float32, 1)
    if colmax.numel() != k:
        raise ValueError("colmax must have one entry per column")
    with _dev(x):
        _lib.check(_lib.load().mp_colmax_abs(x2.data_ptr(), _DT3[x.dtype], x2.shape[0], k, int(acc),
                                             colmax.data_ptr(), _stream()), "mp_colmax_abs")
    return colmax


def smooth_scales(act_max: torch.Tensor, w_colmax: torch.Tensor, alpha: float, dtype: torch.dtype) -> torch.Tensor:
    """``(a^alpha / w^(1-alpha)).clamp(1e-5)`` in ``dtype`` from the fp32 statistics (GPU vectors)."""
    _need(act_max, "act_max", torch.float32, 1)
    _need(w_colmax, "w_colmax", torch.float32, 1)
    if act_max.numel() != w_colmax.numel():
        raise ValueError("act_max and w_colmax differ in length")
    if dtype not in _DT3:
        raise RuntimeError(f"smoothing scales in fp16, bf16 or fp32, got {dtype}")
    out = torch.empty(act_max.numel(), dtype=dtype, device=act_max.device)
    with _dev(act_max):
        _lib.check(_lib.load().mp_smooth_scales(act_max.data_ptr(), w_colmax.data_ptr(), act_max.numel(),
                                                float(alpha), _DT3[dtype], out.data_ptr(), _stream()),
                   "mp_smooth_scales")
    return out


def scale_columns_(w: torch.Tensor, scales: torch.Tensor, divide: bool = False) -> torch.Tensor:
    """In place ``w *= scales`` (or ``/=``) along the last dimension, rounded to ``w``'s dtype."""
    if w.dtype not in _DT3 or scales.dtype != w.dtype:
        raise RuntimeError("scale_columns_ needs w and scales of one dtype among fp16, bf16, fp32")
    if not w.is_cuda or not w.is_contiguous():
        raise RuntimeError("scale_columns_ takes a contiguous GPU tensor")
    k = w.shape[-1]
    sc = scales.contiguous()
    if sc.numel() != k:
        raise ValueError("one scale per column")
    with _dev(w):
        _lib.check(_lib.load().mp_scale_columns(w.data_ptr(), _DT3[w.dtype], w.numel() // k, k, sc.data_ptr(),
                                                int(divide), _stream()), "mp_scale_columns")
    return w

