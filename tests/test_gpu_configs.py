"""GPU parity at the benchmark configurations' full layer shapes, checked on sampled outputs.

Shapes: Llama-2-7B prefill and decode linears (K = 4096 / 11008, N = 4096 / 12288 / 22016 and the
32000-row lm_head) and Llama-3-70B decode linears (K = 8192 / 28672, N = 8192 / 10240 / 28672 and
the fused gate/up at 57344 rows), one-row GEMVs, batched rows and M = 2048 prefill tiles.

Method: the weight is quantized on the GPU by ``w4_quantize_awq`` / ``w4_quantize_gptq_rtn`` (both
bit-exact to the reference's own vectors in test_gpu_parity).  The full-shape kernel then runs, and
for a sample of output columns (48 random ones plus the first and last 16, which hold the tile
tails) the oracle dequantizes those weight rows' codes and forms ``F.linear``'s fp32-accumulated
product.  Bar: relative Frobenius error <= 1e-3 over the sampled columns, every row of M.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import quant as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _ops():
    from mindpipe_amd import ops
    return ops


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _np(t):
    return t.detach().cpu().numpy()


def _rel(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-30))


def _quant_gpu(n, k, seed, zp):
    """fp16 weight N(0, 0.02) quantized on the GPU: (packed int32 [n, k/8], scales, zeros or None)."""
    ops = _ops()
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = (torch.randn(n, k, generator=g, device=DEV) * 0.02).half()
    if zp:
        packed, s, z, _ = ops.w4_quantize_awq(w, 128, True, return_deq=False)
    else:
        _, packed, s = ops.w4_quantize_gptq_rtn(w, 128)
        z = None
    del w
    return packed, s, z


def _cols(n, seed, count=48):
    rng = np.random.default_rng(seed)
    c = set(rng.choice(n, size=min(n, count), replace=False).tolist())
    c |= set(range(min(16, n))) | set(range(max(0, n - 16), n))
    return np.array(sorted(c))


def _x(m, k, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randn(m, k, generator=g, device=DEV).half()


def _ref_cols(x, packed, s, z, cols, k, bias=None):
    """Oracle product for the output columns ``cols``: dequant of those weight rows, then F.linear."""
    idx = torch.as_tensor(cols, device=DEV)
    deq = O.dequant_w4_fp16(_np(packed[idx]), _np(s[idx]), None if z is None else _np(z[idx]), k, 128)
    return O.w4a16_linear(_np(x), deq, None if bias is None else _np(bias[idx]))


# (m, n, k): 70B decode GEMVs and batched rows, 7B decode and prefill linears, the lm_head
W4_FULL = [
    (1, 28672, 8192), (1, 8192, 28672), (1, 10240, 8192), (1, 57344, 8192), (1, 8192, 8192),
    (16, 10240, 8192), (64, 28672, 8192), (16, 8192, 28672), (64, 57344, 8192),
    (1, 12288, 4096), (1, 22016, 4096), (1, 4096, 11008), (8, 22016, 4096), (32, 12288, 4096),
    (2048, 12288, 4096), (2048, 22016, 4096), (2048, 4096, 4096), (2048, 4096, 11008),
    (1, 32000, 4096), (16, 32000, 4096), (2048, 32000, 4096),
]


@pytest.mark.parametrize("m,n,k", W4_FULL)
def test_w4a16_full_shape_sampled(m, n, k):
    _say("w4a16 full", m, n, k)
    ops = _ops()
    zp = (m + n) % 2 == 0 or m == 1  # AWQ zero points on most, the symmetric export on the rest
    packed, s, z = _quant_gpu(n, k, seed=m + n + k, zp=zp)
    x = _x(m, k, seed=7)
    bias = (torch.randn(n, generator=torch.Generator(device=DEV).manual_seed(3), device=DEV) * 0.1).half()
    y = ops.w4a16_gemm(x, packed, s, z, 128, bias)
    torch.cuda.synchronize()
    cols = _cols(n, seed=n)
    ref = _ref_cols(x, packed, s, z, cols, k, bias)
    assert _rel(_np(y)[:, cols], ref) <= 1e-3


@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (1, 28672, 8192)])
def test_w4a16_full_shape_symmetric_and_awq_agree_with_oracle(m, n, k):
    """Both zero-point forms on the same shape (the one-row GEMV paths at K = 4096 and 8192)."""
    _say("w4a16 full zp/sym", m, n, k)
    ops = _ops()
    x = _x(m, k, seed=11)
    for zp in (True, False):
        packed, s, z = _quant_gpu(n, k, seed=5, zp=zp)
        y = ops.w4a16_gemm(x, packed, s, z, 128, None)
        cols = _cols(n, seed=1)
        assert _rel(_np(y)[:, cols], _ref_cols(x, packed, s, z, cols, k)) <= 1e-3


# bf16 (Llama-3 checkpoints are bf16): one-row and batched decode shapes of the 70B / 7B layers and
# 7B prefill linears at M = 2048
W4_BF16_FULL = [(1, 28672, 8192), (1, 8192, 28672), (16, 10240, 8192), (16, 8192, 28672), (1, 57344, 8192),
                (1, 4096, 11008), (8, 22016, 4096), (16, 4096, 4096), (64, 28672, 8192), (2048, 12288, 4096),
                (2048, 4096, 11008)]


@pytest.mark.parametrize("m,n,k", W4_BF16_FULL)
def test_w4a16_bf16_full_shape_sampled(m, n, k):
    """bf16 weight N(0, 0.02) quantized on the GPU in bf16 arithmetic (AWQ, asymmetric on most shapes
    and the symmetric export on the rest); the oracle's bf16 dequant of the sampled rows' codes, then
    F.linear (fp32 accumulation, one bf16 rounding).  Bar: rel. Frobenius error <= 1e-3."""
    _say("w4a16 bf16 full", m, n, k)
    ops = _ops()
    zp = (m + n) % 2 == 0
    g = torch.Generator(device=DEV).manual_seed(m + n + k)
    w = (torch.randn(n, k, generator=g, device=DEV) * 0.02).bfloat16()
    packed, s, z, _ = ops.w4_quantize_awq(w, 128, zp, return_deq=False)
    del w
    x = torch.randn(m, k, generator=torch.Generator(device=DEV).manual_seed(7), device=DEV).bfloat16()
    bias = (torch.randn(n, generator=torch.Generator(device=DEV).manual_seed(3), device=DEV) * 0.1).bfloat16()
    y = ops.w4a16_gemm(x, packed, s, z, 128, bias)
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16
    cols = _cols(n, seed=n)
    idx = torch.as_tensor(cols, device=DEV)
    bits = lambda t: _np(t.view(torch.int16)).view(np.uint16)  # noqa: E731
    deq = O.dequant_w4_bf16(_np(packed[idx]), bits(s[idx]), None if z is None else bits(z[idx]), k, 128)
    ref = O.bf16_bits_to_f32(O.w4a16_linear(bits(x), deq, bits(bias[idx]), dtype="bf16"))
    assert _rel(_np(y.float())[:, cols], ref) <= 1e-3


# fused gate/up: [2I, K] with the gate rows first; 70B (I = 28672) and 7B (I = 11008)
SWIGLU_FULL = [(1, 28672, 8192), (16, 28672, 8192), (1, 11008, 4096), (8, 11008, 4096)]


@pytest.mark.parametrize("m,i,k", SWIGLU_FULL)
def test_w4a16_swiglu_full_shape_sampled(m, i, k):
    """``silu(G) * U`` of the fused gate/up GEMM against the oracle's dequant -> matmul (fp16 G, U) ->
    SiLU-mul on sampled intermediate columns."""
    _say("w4a16 swiglu full", m, i, k)
    ops = _ops()
    packed, s, z = _quant_gpu(2 * i, k, seed=i + k, zp=True)
    x = _x(m, k, seed=9)
    act = ops.w4a16_gemm_swiglu(x, packed, s, z, 128, None)
    torch.cuda.synchronize()
    cols = _cols(i, seed=i)
    g = _ref_cols(x, packed, s, z, cols, k).astype(np.float32)
    u = _ref_cols(x, packed, s, z, cols + i, k).astype(np.float32)
    ref = (g / (1.0 + np.exp(-g)) * u).astype(np.float16)
    assert _rel(_np(act)[:, cols], ref) <= 1e-3
