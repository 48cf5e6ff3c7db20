"""CPU oracle: a numpy restatement of MindPipe's quantized-linear arithmetic.

TEST INFRASTRUCTURE ONLY.  Nothing in ``mindpipe_amd`` may import this module;
it is imported by ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``, always as the checker (or the timed CPU
baseline), never as the product path.

Conventions
-----------
* Every fp16 tensor op of the reference is restated as "compute in float32,
  round once to float16", which is what PyTorch does for ``torch.half`` on the
  CPU and the GPU.  ``_h(x)`` is that rounding.
* ``torch.round`` is round-half-to-even; ``np.rint`` is the same.
* bf16 is carried as uint16 bit patterns (numpy has no bfloat16):
  ``f32_to_bf16_bits`` rounds to nearest-even, ``bf16_bits_to_f32`` widens.

Pinning (how each function is checked; see ``tests/test_oracle.py``)
--------------------------------------------------------------------
* ``pack_int4_signed`` / ``unpack_int4_signed``: the reference's own known
  answers (pack KAT, export KAT) plus a brute-force bit loop.
* ``quantize_weight_per_channel_export``: the reference's tiny-Qwen2 export
  fixture values (including the 63.5 / -63.5 ties).
* ``pseudo_quantize_tensor``: the reference's own outputs (fp16: asym, per-row
  fallback, sym; bf16: asym with a constant group, sym), invariants fixed by the
  definition (codes in [0,15], group min/max map to codes 0/15 up to one
  rounding step), a hand-computed case, and a float64 brute force.
* ``quantize_activation_per_token_fake`` / ``quantize_weight_per_channel_fake``:
  the reference's own outputs in fp16 and bf16.
* ``w8a8_linear_fake``: the reference ``SmoothQuantLinear`` forward (fp16, bf16,
  with and without the output fake-quant), bit-exact.
* ``compute_smooth_scales``: the reference ``_compute_smooth_scales`` (fp16,
  bf16, with a clamped column), bit-exact, plus a closed form.
* ``moe_fake``: the reference ``SmoothQuantPackedMoeExperts`` forward (fp16,
  bf16, with an all-zero token and a one-token expert), bit-exact, and a planted
  mistake (gate/up swapped) that lands far from it.
* ``gptq_rtn_quantize``: the reference's GPTQ reconstruction invariant
  (int in [-8,7], int*scale reproduces the fake-quant weight) and hand cases
  (all-positive rows keep xmin = 0).
* per-token quantizers: closed form checks (max |q| == 127 on every non-zero
  row, |x - q*s| <= s/2, ties to even) and brute-force Python loops on small
  rows.
* ``w8a8_linear_runtime``: exact int64 brute force on tiny inputs.
* ``dense_mlp_runtime``: equals ``moe_runtime`` with one expert at one chunk.
* ``add_rms_norm_quant``: closed forms (constant rows, +-a rows), scale
  invariance, the residual identity and q == per-token quant of y.
* MoE: a brute-force per-assignment loop on tiny E/T/H/I, routing invariants.
Nothing here is "parity unpinned" except where a docstring says so.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "f32_to_bf16_bits",
    "bf16_bits_to_f32",
    "pseudo_quantize_tensor",
    "gptq_rtn_quantize",
    "pack_int4_signed",
    "unpack_int4_signed",
    "pack_uint4",
    "unpack_uint4",
    "dequant_w4_fp16",
    "dequant_w4_export_fp32",
    "w4a16_linear",
    "quantize_activation_per_token_fake",
    "quantize_weight_per_channel_fake",
    "quantize_per_token_runtime",
    "add_rms_norm_quant",
    "dense_mlp_runtime",
    "quantize_weight_per_channel_export",
    "w8a8_linear_runtime",
    "w8a8_linear_fake",
    "compute_smooth_scales",
    "mixtral_router",
    "moe_runtime",
    "moe_fake",
    "int_matmul_nt",
]


# ---------------------------------------------------------------- rounding helpers
def _h(x) -> np.ndarray:
    """Round float32 values once to float16 (PyTorch half-op semantics)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16)


def _f(x) -> np.ndarray:
    return np.asarray(x).astype(np.float32)


def f32_to_bf16_bits(x) -> np.ndarray:
    """float32 -> bfloat16 bit pattern, round-to-nearest-even, NaN kept quiet."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    rounded = np.where(nan, (b >> 16) | 0x40, rounded)
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def _round_to(x, dt: str) -> np.ndarray:
    """float32 values rounded once to ``dt`` ("fp16" / "bf16"), returned as float32
    (the value PyTorch keeps after one op in that dtype)."""
    x = np.asarray(x, dtype=np.float32)
    if dt == "fp16":
        return x.astype(np.float16).astype(np.float32)
    if dt == "bf16":
        return bf16_bits_to_f32(f32_to_bf16_bits(x))
    raise ValueError(dt)


def _bits_out(x32: np.ndarray, dt: str) -> np.ndarray:
    """float32 values that are exact in ``dt`` -> an fp16 array or bf16 uint16 bits."""
    return np.asarray(x32, np.float32).astype(np.float16) if dt == "fp16" else f32_to_bf16_bits(x32)


def _to_out(y_f32: np.ndarray, out_dtype: str) -> np.ndarray:
    if out_dtype == "fp16":
        return y_f32.astype(np.float16)
    if out_dtype == "bf16":
        return f32_to_bf16_bits(y_f32)
    if out_dtype == "fp32":
        return y_f32.astype(np.float32)
    raise ValueError(out_dtype)


def _in_f32(x: np.ndarray, in_dtype: str) -> np.ndarray:
    if in_dtype == "bf16":
        return bf16_bits_to_f32(x)
    return _f(x)


# ---------------------------------------------------------------- W4 (AWQ / GPTQ)
def pseudo_quantize_tensor(w, n_bit=4, zero_point=True, q_group_size=128, dtype="fp16"):
    """AWQ pseudo-quantization in the arithmetic of the weight dtype (fp16 or bf16).

    Follows ``algorithm/quantization/ptq/awq/source/awq/quantize/quantizer.py:63-105``:
    reshape to ``[-1, g]`` (per-row when g does not divide K, ``:67-68``),
    ``s = (max-min).clamp(1e-5) / (2^n-1)``, ``z = clamp(-round(min/s), 0, 2^n-1)``,
    ``q = clamp(round(w/s) + z, 0, 2^n-1)``, ``w_deq = (q - z) * s``, each op rounded
    once to the weight dtype.  ``zero_point=False`` is the symmetric branch
    (``:79-85``): ``s = max|w|.clamp(1e-5)/(2^(n-1)-1)``, codes in
    ``[-2^(n-1), 2^(n-1)-1]``.

    ``dtype="fp16"``: ``w`` is a float16 array and the float outputs are float16.
    ``dtype="bf16"``: ``w`` holds bfloat16 bit patterns (uint16) and so do the outputs.

    Returns ``(w_deq [N,K], scales [N,K/g], zeros [N,K/g] or None, codes uint8/int8 [N,K])``;
    the first three are what ``get_scale_zp=True`` returns.
    """
    if dtype == "fp16":
        wf = _f(np.asarray(w, dtype=np.float16))
    else:
        wf = bf16_bits_to_f32(w)
    if wf.ndim != 2:
        raise ValueError("expected a 2-D weight")
    R = lambda v: _round_to(v, dtype)  # noqa: E731
    n_rows, k = wf.shape
    g = q_group_size
    if g > 0 and k % g != 0:
        g = -1
    wg = wf.reshape(-1, g) if g > 0 else wf
    eps = R(np.float32(1e-5))
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        if zero_point:
            max_val = wg.max(axis=1, keepdims=True)
            min_val = wg.min(axis=1, keepdims=True)
            max_int, min_int = 2**n_bit - 1, 0
            d = R(max_val - min_val)
            d = np.where(d < np.float32(1e-5), eps, d)
            scales = R(d / np.float32(max_int))
            zeros = np.clip(-np.rint(R(min_val / scales)), min_int, max_int).astype(np.float32)
        else:
            max_val = np.abs(wg).max(axis=1, keepdims=True)
            max_val = np.where(max_val < np.float32(1e-5), eps, max_val)
            max_int, min_int = 2 ** (n_bit - 1) - 1, -(2 ** (n_bit - 1))
            scales = R(max_val / np.float32(max_int))
            zeros = np.zeros_like(scales)
        t = np.rint(R(wg / scales))
        q = np.clip(R(t + zeros), min_int, max_int)
        deq = R(R(q - zeros) * scales)
    deq = _bits_out(deq.reshape(n_rows, k), dtype)
    scales_o = _bits_out(scales.reshape(n_rows, -1), dtype)
    codes = q.reshape(n_rows, k).astype(np.int16)
    if zero_point:
        return deq, scales_o, _bits_out(zeros.reshape(n_rows, -1), dtype), codes.astype(np.uint8)
    return deq, scales_o, None, codes.astype(np.int8)


def gptq_rtn_quantize(w, bits=4, groupsize=128):
    """Round-to-nearest GPTQ symmetric group quantizer in float32.

    ``Quantizer.find_params(weight=True)`` with ``perchannel=True, sym=True``
    (``algorithm/quantization/ptq/gptq/source/quant.py:44-82``) applied per group
    of ``groupsize`` columns, then ``quantize_with_qint`` (``quant.py:13-17``) and
    the signed export ``q - zero`` (``gptq.py:157-161``), scale stored fp16
    (``gptq/method.py:344``).  This is the artifact GPTQ produces with no Hessian
    error feedback (its RTN special case).

    Returns ``(int_weight int8 [N,K] in [-8,7], scale fp16 [N,K/g], w_fake fp32 [N,K])``.
    """
    w = _f(w)
    n_rows, k = w.shape
    g = k if groupsize in (-1, 0) else groupsize
    if k % g:
        raise ValueError("groupsize must divide K")
    maxq = np.float32(2**bits - 1)
    ng = k // g
    int_w = np.empty((n_rows, k), np.int8)
    scale = np.empty((n_rows, ng), np.float32)
    fake = np.empty((n_rows, k), np.float32)
    for gi in range(ng):
        x = w[:, gi * g:(gi + 1) * g]
        xmin = np.minimum(x.min(axis=1), np.float32(0))
        xmax = np.maximum(x.max(axis=1), np.float32(0))
        xmax = np.maximum(np.abs(xmin), xmax)
        xmin = np.where(xmin < 0, -xmax, xmin)
        both0 = (xmin == 0) & (xmax == 0)
        xmin = np.where(both0, np.float32(-1), xmin)
        xmax = np.where(both0, np.float32(1), xmax)
        s = ((xmax - xmin) / maxq).astype(np.float32)
        zero = np.float32((maxq + 1) / 2)
        q = np.clip(np.rint(x / s[:, None]) + zero, 0, maxq).astype(np.float32)
        int_w[:, gi * g:(gi + 1) * g] = (q - zero).astype(np.int8)
        scale[:, gi] = s
        fake[:, gi * g:(gi + 1) * g] = s[:, None] * (q - zero)
    return int_w, scale.astype(np.float16), fake


def pack_int4_signed(int_weight) -> np.ndarray:
    """``pack_int4_for_vllm`` (``algorithm/quantization/exporters/vllm.py:89-111``).

    ``u = int + 8``; column k goes to nibble ``k % 8`` of int32 word ``k // 8``;
    K is zero-padded (u = 0) to a multiple of 8.  Range [-8, 7] is enforced.
    """
    iw = np.asarray(int_weight)
    if iw.ndim != 2:
        raise ValueError(f"Expected 2D int_weight, got shape {iw.shape}.")
    if iw.size and (iw.min() < -8 or iw.max() > 7):
        raise ValueError("int4 weights must be in signed range [-8, 7].")
    return pack_uint4((iw.astype(np.int16) + 8).astype(np.uint8))


def pack_uint4(codes) -> np.ndarray:
    """Pack unsigned 4-bit codes (AWQ asymmetric ``q``) in the same nibble order."""
    u = np.asarray(codes).astype(np.uint32)
    if u.size and u.max() > 15:
        raise ValueError("uint4 codes must be in [0, 15]")
    n_rows, k = u.shape
    words = -(-k // 8)
    pad = words * 8 - k
    if pad:
        u = np.pad(u, [(0, 0), (0, pad)])
    packed = np.zeros((n_rows, words), np.uint32)
    for o in range(8):
        packed |= u[:, o::8] << np.uint32(4 * o)
    return np.ascontiguousarray(packed).view(np.int32)


def unpack_uint4(packed, k) -> np.ndarray:
    p = np.asarray(packed, dtype=np.int32).view(np.uint32)
    out = np.empty((p.shape[0], p.shape[1] * 8), np.uint8)
    for o in range(8):
        out[:, o::8] = (p >> np.uint32(4 * o)) & np.uint32(0xF)
    return out[:, :k]


def unpack_int4_signed(packed, k) -> np.ndarray:
    """Inverse of ``pack_int4_signed`` (``tests/test_vllm_real_quant_export.py:23-27``)."""
    return (unpack_uint4(packed, k).astype(np.int16) - 8).astype(np.int8)


def dequant_w4_fp16(packed, scales, zeros, k, group_size):
    """fp16 dequant ``(u - z) * s`` with each op rounded to fp16.

    ``zeros=None`` means the symmetric export (stored nibble = int + 8, so z = 8),
    which is the same arithmetic as AWQ's ``(q - z) * s``
    (``quantizer.py:89-96``) with a constant zero point.
    """
    u = unpack_uint4(packed, k).astype(np.float32)
    n_rows = u.shape[0]
    s = np.repeat(_f(scales), group_size, axis=1)[:, :k]
    if zeros is None:
        z = np.full((n_rows, k), 8.0, np.float32)
    else:
        z = np.repeat(_f(zeros), group_size, axis=1)[:, :k]
    return _h(_f(_h(u - z)) * s)


def dequant_w4_bf16(packed, scales, zeros, k, group_size):
    """bf16 dequant ``R(R(u - z) * s)`` from the packed codes, the weight that AWQ's
    ``pseudo_quantize_tensor`` returns in bf16 (``quantizer.py:95-105``: ``(q - zeros) * scales``,
    each op rounded to bf16; ``R(u - z)`` is exact).  ``scales`` / ``zeros`` are bf16 bit patterns;
    ``zeros=None`` is the symmetric export (stored nibble = int + 8, so z = 8).  Returns bf16 bits."""
    u = unpack_uint4(packed, k).astype(np.float32)
    n_rows = u.shape[0]
    s = np.repeat(bf16_bits_to_f32(scales), group_size, axis=1)[:, :k]
    if zeros is None:
        z = np.full((n_rows, k), 8.0, np.float32)
    else:
        z = np.repeat(bf16_bits_to_f32(zeros), group_size, axis=1)[:, :k]
    return f32_to_bf16_bits(_round_to(u - z, "bf16") * s)


def dequant_w4_export_fp32(packed, scale, weight_shape):
    """``_dequantize_weight`` (``scripts/repro/evaluate_real_quant_export_dequant.py:46-64``):
    signed ints times the fp16 scale, in float32."""
    rows, cols = (int(v) for v in weight_shape)
    iw = unpack_int4_signed(packed, cols).astype(np.float32)
    g = cols // scale.shape[1]
    return iw * np.repeat(_f(scale), g, axis=1)[:, :cols]


def w4a16_linear(x, w_deq, bias=None, dtype="fp16"):
    """``F.linear(x, w_deq, bias)`` on fp16 (or bf16 bit-pattern) operands: fp32 accumulation,
    one rounding to the dtype."""
    y = _in_f32(x, dtype) @ _in_f32(w_deq, dtype).T
    if bias is not None:
        y = y + _in_f32(bias, dtype)
    return _to_out(y.astype(np.float32), dtype)


# ---------------------------------------------------------------- W8A8 (SmoothQuant)
def quantize_activation_per_token_fake(x, n_bits=8, dtype="fp16"):
    """``quantize_activation_per_token_absmax`` in the arithmetic of ``x``'s dtype
    (``algorithm/quantization/ptq/smoothquant/source/smoothquant/fake_quant.py:22-31``):
    ``s = (max|x|).clamp(1e-5) / 127``, ``fake = round(x / s) * s``, each op rounded once.

    ``dtype="fp16"``: float16 arrays in and out.  ``dtype="bf16"``: bfloat16 bit patterns
    (uint16) in and out.  Returns ``(codes int16, scale [M], fake)``: the integer codes
    ``round(x / s)``, in [-127, 127] for fp16 and [-128, 128] for bf16 (``r(x / s)`` can reach
    127.5 when the bf16 scale rounds down).
    """
    xf = _f(np.asarray(x, dtype=np.float16)) if dtype == "fp16" else bf16_bits_to_f32(x)
    R = lambda v: _round_to(v, dtype)  # noqa: E731
    q_max = np.float32(2 ** (n_bits - 1) - 1)
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        s = np.abs(xf).max(axis=-1, keepdims=True)
        s = np.where(s < np.float32(1e-5), R(np.float32(1e-5)), s)
        s = R(s / q_max)
        q = np.rint(R(xf / s))
        fake = R(q * s)
    return q.astype(np.int16), _bits_out(s[..., 0], dtype), _bits_out(fake, dtype)


def quantize_weight_per_channel_fake(w, n_bits=8, dtype="fp16"):
    """``quantize_weight_per_channel_absmax`` (``fake_quant.py:10-19``): the same
    arithmetic as the activation quantizer along the last dim."""
    return quantize_activation_per_token_fake(w, n_bits, dtype)


def quantize_per_token_runtime(x, in_dtype="fp16"):
    """Per-token dynamic int8 quant with an fp32 scale: the runtime contract of
    ``npu_dynamic_quant`` (``vllm_ascend.patch:3950``; ``scale = absmax / 127`` per
    ``vllm_ascend.patch:1741``; int8 codes + fp32 ``[T]`` scale, ``:3961-3962``).

    ``s = fp32(absmax) / 127``; ``q = clamp(rint(x / s), -127, 127)``; an all-zero
    row gives ``s = 0`` and ``q = 0``.  The arithmetic inside the Ascend op is not
    published, so the division form is this build's definition (parity of the
    NPU op itself is unpinned; the GPU kernel is pinned to this function).
    """
    xf = _in_f32(x, in_dtype)
    amax = np.abs(xf).max(axis=-1)
    s = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        q = np.rint(xf / s[..., None])
    q = np.where(s[..., None] == 0, 0, q)
    q = np.clip(q, -127, 127).astype(np.int8)
    return q, s


def add_rms_norm_quant(x, residual, weight, eps, in_dtype="fp16", quant=True):
    """Residual add + RMSNorm + per-token dynamic int8 quant: the chain the W8A8
    runtime runs in front of qkv / gate_up (``vllm_ascend.patch:746-787``:
    ``npu_add_rms_norm_dynamic_quant``, or ``npu_add_rms_norm`` then the linear's
    ``npu_dynamic_quant``).  The Ascend ops are closed; the RMSNorm arithmetic
    restated here is vLLM's native RMSNorm (third-party, not under the reference;
    vLLM 0.11 is named by ``acceleration/README.md:10-11``):

    * ``sum = fp32(x) + fp32(residual)``; ``residual_out = round(sum)``
    * ``var = mean(sum**2)`` (fp32), ``rstd = 1 / sqrt(var + eps)``
    * ``y = round(round(sum * rstd) * weight)`` (rounding to the input dtype twice:
      ``x.to(orig_dtype)`` then ``* self.weight`` in that dtype)
    * ``q, s = quantize_per_token_runtime(y)``

    Pinned by closed forms (constant rows, +-a rows), RMSNorm scale invariance,
    the residual identity ``f(x, r) == f(x + r, None)`` for exact sums, and the
    identity ``q == quantize_per_token_runtime(y)``; the fp32 summation order of
    ``mean`` is not fixed by any of them (a 1-ulp difference of ``y`` is allowed).
    Returns ``(y, q, s, residual_out)`` (``q``/``s`` None unless ``quant``;
    ``residual_out`` None without a residual).
    """
    xf = _in_f32(x, in_dtype)
    if residual is not None:
        xf = (xf + _in_f32(residual, in_dtype)).astype(np.float32)
    rout = _to_out(xf, in_dtype) if residual is not None else None
    var = (np.square(xf.astype(np.float64)).mean(axis=-1)).astype(np.float32)
    rstd = (np.float32(1.0) / np.sqrt(var + np.float32(eps))).astype(np.float32)
    yn = _in_f32(_to_out((xf * rstd[..., None]).astype(np.float32), in_dtype), in_dtype)
    w = _in_f32(np.asarray(weight), in_dtype)
    y = _to_out((yn * w).astype(np.float32), in_dtype)
    if not quant:
        return y, None, None, rout
    q, sc = quantize_per_token_runtime(y, in_dtype)
    return y, q, sc, rout


def quantize_weight_per_channel_export(w, in_dtype="fp16"):
    """Real-export W8 quantizer ``quantize_weight_per_channel``
    (``scripts/repro/export_fp16_to_ascend_w8a8_dynamic_probe.py:175-195``; same as
    ``export_qwen3_moe_fp16_to_ascend_w8a8_dynamic.py:187-205``).

    fp32 math: ``s = max|w| / 127`` clamped at 1e-8, ``q = round(w/s).clamp(-127,127)``.
    Returns ``(q int8 [N,K], s_fp32 [N], s_src [N] in the source dtype, offset zeros)``.
    """
    wf = _in_f32(w, in_dtype)
    if not np.isfinite(wf).all():
        raise ValueError("Source weight contains non-finite values")
    s = (np.abs(wf).max(axis=1) / np.float32(127.0)).astype(np.float32)
    s = np.maximum(s, np.float32(1e-8))
    q = np.clip(np.rint(wf / s[:, None]), -127, 127).astype(np.int8)
    s_src = f32_to_bf16_bits(s) if in_dtype == "bf16" else s.astype(np.float16)
    return q, s, s_src, np.zeros_like(s_src)


def int_matmul_nt(a, b) -> np.ndarray:
    """Exact ``a @ b.T`` for int8 operands (int64 result).

    Uses float64 BLAS: every product is <= 127*128 and K <= 2^20, so every
    partial sum is an integer below 2^53 and float64 represents it exactly.
    """
    a = np.asarray(a)
    b = np.asarray(b)
    if a.shape[-1] > (1 << 20):
        raise ValueError("K too large for the exact float64 path")
    af = a.astype(np.float64)
    out = np.empty((a.shape[0], b.shape[0]), np.int64)
    step = max(1, (64 << 20) // max(1, 8 * b.shape[1]))  # ~64 MB of float64 weight rows at a time
    for r0 in range(0, b.shape[0], step):
        out[:, r0:r0 + step] = np.rint(af @ b[r0:r0 + step].astype(np.float64).T).astype(np.int64)
    return out


def w8a8_linear_runtime(qx, s_tok, qw, s_ch, bias=None, out_dtype="fp16", bias_dtype="fp16"):
    """``npu_quant_matmul`` contract (``vllm_ascend.patch:4007-4015``):
    ``int32 acc = qx . qw^T``, ``y = (acc * s_tok[m]) * s_ch[n] (+ bias[n])`` in
    float32, rounded once to ``out_dtype``.  The multiplication order is this
    build's definition; the GPU epilogue uses the same order, so results are
    bit-identical.
    """
    acc = int_matmul_nt(qx, qw)
    if np.abs(acc).max(initial=0) >= 2**31:
        raise OverflowError("int32 accumulator overflow")
    y = (acc.astype(np.float32) * _f(s_tok)[:, None]).astype(np.float32)
    y = (y * _f(s_ch)[None, :]).astype(np.float32)
    if bias is not None:
        y = (y + _in_f32(bias, bias_dtype)[None, :]).astype(np.float32)
    return _to_out(y, out_dtype)


def w8a8_linear_fake(x, w, bias=None, dtype="fp16"):
    """``SmoothQuantLinear.forward`` fake path (``fake_quant.py:85-88``):
    ``F.linear(fq_token(x), fq_channel(w), b)`` with fp32 accumulation and one rounding to
    ``dtype``; ``w`` is the float weight before ``from_float`` (which applies
    ``quantize_weight_per_channel_absmax``, ``:110``).  fp16 arrays, or bf16 bit patterns
    for ``dtype="bf16"``."""
    _, _, xq = quantize_activation_per_token_fake(x, 8, dtype)
    _, _, wq = quantize_weight_per_channel_fake(w, 8, dtype)
    y = _in_f32(xq, dtype) @ _in_f32(wq, dtype).T
    if bias is not None:
        y = y + _in_f32(bias, dtype)
    return _to_out(y.astype(np.float32), dtype)


def compute_smooth_scales(act_max, weights, alpha=0.5, dtype="fp16"):
    """``_compute_smooth_scales`` (``smoothquant/smooth.py:7-25``):
    ``s_j = (a_j^alpha / w_j^(1-alpha)).clamp(1e-5)`` in the weight dtype, where
    ``a_j`` is the calibration abs-max (fp32) cast to that dtype and
    ``w_j = max_n |W_nj|`` (max over every fc sharing the norm, clamped at 1e-5).
    fp16 arrays, or bf16 bit patterns (weights and result) for ``dtype="bf16"``."""
    R = lambda v: _round_to(v, dtype)  # noqa: E731
    a = R(np.asarray(act_max, dtype=np.float32))
    if not isinstance(weights, (list, tuple)):
        weights = [weights]
    wmax = np.max(np.stack([np.abs(_in_f32(np.asarray(w), dtype)).max(axis=0) for w in weights]), axis=0)
    wmax = np.where(wmax < np.float32(1e-5), R(np.float32(1e-5)), wmax)
    # the fp32 powers taken correctly rounded (float64 power, rounded to float32): torch's x.pow(0.5) is
    # a square root, which is; other exponents go through the platform's powf, faithful to an ulp but
    # not correctly rounded (numpy's float32 power differs from the correctly rounded value in about
    # 20% of entries here), so the correctly rounded value is the one definition every platform nears
    e1, e2 = np.float64(np.float32(alpha)), np.float64(np.float32(1 - alpha))
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        num = R(np.power(a.astype(np.float64), e1).astype(np.float32))
        den = R(np.power(wmax.astype(np.float64), e2).astype(np.float32))
        sc = R(num / den)
    sc = np.where(sc < np.float32(1e-5), R(np.float32(1e-5)), sc)
    return _bits_out(sc, dtype)


# ---------------------------------------------------------------- MoE
def mixtral_router(logits, top_k=2):
    """HF ``MixtralTopKRouter.forward`` after the router linear (transformers
    ``models/mixtral/modeling_mixtral.py:104-112``; third-party, not under the
    reference tree): fp32 softmax, top-k, renormalise.  Ties resolve to the
    lower expert index.  Parity with torch.topk's tie order: unpinned (ties have
    probability zero on continuous inputs)."""
    lf = _f(logits)
    e = np.exp(lf - lf.max(axis=-1, keepdims=True))
    p = e / e.sum(axis=-1, keepdims=True)
    idx = np.argsort(-p, axis=-1, kind="stable")[:, :top_k].astype(np.int32)
    w = np.take_along_axis(p, idx, axis=-1)
    w = (w / w.sum(axis=-1, keepdims=True)).astype(np.float32)
    return idx, w


def _silu(g):
    return (g / (np.float32(1.0) + np.exp(-g))).astype(np.float32)


def moe_runtime(x, topk_ids, topk_w, qw13, s13, qw2, s2, out_dtype="fp16", return_intermediate=False):
    """Runtime-semantic W8A8 MoE chain (the contract of ``_run_expert_tile``,
    ``vllm_ascend.patch:2356-2423``, and the C++ bridge
    ``aclnn_grouped_swiglu_out_bridge.cpp:157-273``):

    1. per-token int8 quant of ``x`` (fp32 scale);
    2. GMM1 per assignment ``acc = qx . qw13[e]^T``; ``g = (acc*s_x)*s13[e]``;
       ``h = silu(g[:, :I]) * g[:, I:]`` (gate first, ``chunk(2)`` order of
       ``fake_quant.py:181``); per-row int8 requant of ``h`` (fp32 scale);
    3. GMM2 ``y = (acc2*s_h)*s2[e]``;
    4. combine ``out[t] = sum_j w[t,j] * y[t,j]`` in fp32, rounded once.

    Weights use the module layout: ``qw13 [E, 2I, H]``, ``qw2 [E, H, I]``
    (``fake_quant.py:140-142``), per-row scales ``s13 [E, 2I]``, ``s2 [E, H]``.
    silu's exp is not correctly rounded on either side, so a requant code may
    differ by one where ``h/s`` lands within an ulp of a .5 boundary.
    """
    x = np.asarray(x)
    t_count, hdim = x.shape
    top_k = topk_ids.shape[1]
    inter = qw2.shape[2]
    qx, sx = quantize_per_token_runtime(x)
    y_assign = np.zeros((t_count, top_k, hdim), np.float32)
    qh_all = {}
    for e in range(qw13.shape[0]):
        tok, pos = np.nonzero(topk_ids == e)
        if tok.size == 0:
            continue
        acc = int_matmul_nt(qx[tok], qw13[e])
        g = ((acc.astype(np.float32) * sx[tok][:, None]).astype(np.float32) * _f(s13[e])[None, :]).astype(np.float32)
        h = (_silu(g[:, :inter]) * g[:, inter:]).astype(np.float32)
        qh, sh = quantize_per_token_runtime(h, in_dtype="fp32")
        acc2 = int_matmul_nt(qh, qw2[e])
        y = ((acc2.astype(np.float32) * sh[:, None]).astype(np.float32) * _f(s2[e])[None, :]).astype(np.float32)
        y_assign[tok, pos] = y
        qh_all[e] = (tok, pos, qh, sh)
    out = np.zeros((t_count, hdim), np.float32)
    for j in range(top_k):
        out = (out + _f(topk_w[:, j])[:, None] * y_assign[:, j]).astype(np.float32)
    res = _to_out(out, out_dtype)
    if return_intermediate:
        return res, qh_all
    return res


def dense_mlp_runtime(x, qw13, s13, qw2, s2, chunks=1, out_dtype="fp16", qx=None, sx=None):
    """Dense-MLP W8A8 chain of the reference's chunked Qwen2 MLP
    (``vllm.patch:883-1037``; weight split ``vllm_ascend.patch:4149-4277``):
    per-token quant of ``x`` (or a given ``(qx, sx)``), then for each of ``chunks``
    slices of the intermediate dimension the grouped GEMM1 + SwiGLU + requant
    (``npu_grouped_matmul_swiglu_quant`` with one group of all tokens) on the gate
    rows ``[c*cs, (c+1)*cs)`` and the matching up rows, the down GEMM on the same
    slice of the down weight's columns, and the fp32 sum over chunks
    (``npu_quant_matmul_reduce_sum``, down scale rounded to bf16), rounded once.
    With ``chunks == 1`` this is the single-chunk path (``npu_quant_matmul`` on the
    requantized hidden state, fp32 down scale; ``vllm.patch:1003-1037``).
    ``qw13 [2I, H]`` (gate rows first), ``s13 [2I]``, ``qw2 [H, I]``, ``s2 [H]``.
    Pinned: ``chunks == 1`` equals ``moe_runtime`` with one expert, top-1, weight 1
    (a separate code path); the integer products are exact."""
    if qx is None:
        qx, sx = quantize_per_token_runtime(x)
    inter = qw2.shape[1]
    cs = inter // chunks
    # the chunked path's down scale is rounded to bf16 (vllm_ascend.patch:4262-4264)
    s2c = _f(s2) if chunks == 1 else bf16_bits_to_f32(f32_to_bf16_bits(_f(s2)))
    out = np.zeros((qx.shape[0], qw2.shape[0]), np.float32)
    for c in range(chunks):
        rows = np.r_[c * cs:(c + 1) * cs, inter + c * cs:inter + (c + 1) * cs]
        acc = int_matmul_nt(qx, qw13[rows])
        g = ((acc.astype(np.float32) * sx[:, None]).astype(np.float32) * _f(s13[rows])[None, :]).astype(np.float32)
        h = (_silu(g[:, :cs]) * g[:, cs:]).astype(np.float32)
        qh, sh = quantize_per_token_runtime(h, in_dtype="fp32")
        acc2 = int_matmul_nt(qh, np.ascontiguousarray(qw2[:, c * cs:(c + 1) * cs]))
        y = ((acc2.astype(np.float32) * sh[:, None]).astype(np.float32) * s2c[None, :]).astype(np.float32)
        out = (out + y).astype(np.float32)
    return _to_out(out, out_dtype)


def moe_fake(x, topk_ids, topk_w, gate_up_proj, down_proj, dtype="fp16", prequantized=False):
    """``SmoothQuantPackedMoeExperts`` construction + ``forward`` fake path
    (``fake_quant.py:124-191``) with SiLU: per-channel fake-quant weights
    ``gate_up_proj [E,2I,H]`` / ``down_proj [E,H,I]``; for each hit expert in ascending
    order, per-token fake quant of its tokens, ``F.linear`` (fp32 accumulation, one
    rounding), ``chunk(2)``, ``silu(gate) * up`` (two roundings), per-token fake quant,
    ``F.linear``, times the fp32 router weight (rounded once), ``index_add_`` (one
    rounding per add).  Every rounding is to ``dtype``; fp16 arrays, or bf16 bit
    patterns for ``dtype="bf16"`` (router weights fp32 in both cases).

    ``prequantized=True``: the weights given are already the fake-quant weights (the
    construction step ``:140-142`` done elsewhere), so only the forward is computed.
    Each token's output depends on its own row and experts alone, so the forward may be
    given any subset of the tokens."""
    R = lambda v: _round_to(v, dtype)  # noqa: E731
    F32 = lambda a: _in_f32(np.asarray(a), dtype)  # noqa: E731
    xf = F32(x)
    n_exp = gate_up_proj.shape[0]
    if prequantized:
        wq13 = [F32(gate_up_proj[e]) for e in range(n_exp)]
        wq2 = [F32(down_proj[e]) for e in range(n_exp)]
    else:
        wq13 = [F32(quantize_weight_per_channel_fake(gate_up_proj[e], 8, dtype)[2]) for e in range(n_exp)]
        wq2 = [F32(quantize_weight_per_channel_fake(down_proj[e], 8, dtype)[2]) for e in range(n_exp)]
    out = np.zeros_like(xf)
    inter = down_proj.shape[2]
    for e in range(n_exp):
        top_k_pos, token_idx = np.nonzero((topk_ids == e).T)
        if token_idx.size == 0:
            continue
        cur = F32(quantize_activation_per_token_fake(_bits_out(xf[token_idx], dtype), 8, dtype)[2])
        gu = R(cur @ wq13[e].T)
        gate, up = gu[:, :inter], gu[:, inter:]
        act = R(_silu(gate))
        hcur = R(act * up)
        hcur = F32(quantize_activation_per_token_fake(_bits_out(hcur, dtype), 8, dtype)[2])
        y = R(hcur @ wq2[e].T)
        y = R(y * _f(topk_w[token_idx, top_k_pos])[:, None])
        for r, t in enumerate(token_idx):
            out[t] = R(out[t] + y[r])
    return _bits_out(out, dtype)
