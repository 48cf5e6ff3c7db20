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
# M = 1 / 16 / 64: 70B decode at B = 1 / 16 / 64 (one-row GEMV and batched kernel forms); M = 1 / 8 / 32:
# 7B decode at B = 1 / 8 / 32; M = 2048: the 7B prefill (the prefill kernel's SwiGLU form)
SWIGLU_FULL = [(1, 28672, 8192), (16, 28672, 8192), (64, 28672, 8192), (1, 11008, 4096), (8, 11008, 4096),
               (32, 11008, 4096), (2048, 11008, 4096)]


@pytest.mark.parametrize("dt", ["fp16", "bf16"])
@pytest.mark.parametrize("m,i,k", SWIGLU_FULL)
def test_w4a16_swiglu_full_shape_sampled(m, i, k, dt):
    """``silu(G) * U`` of the fused gate/up GEMM against the oracle's dequant -> matmul (G, U rounded
    to the activation dtype) -> SiLU-mul (silu rounded, then the product) on sampled intermediate
    columns, in fp16 and bf16.  Bar: rel. Frobenius error <= 1e-3."""
    _say("w4a16 swiglu full", m, i, k, dt)
    ops = _ops()
    if dt == "fp16":
        packed, s, z = _quant_gpu(2 * i, k, seed=i + k, zp=True)
        x = _x(m, k, seed=9)
        act = ops.w4a16_gemm_swiglu(x, packed, s, z, 128, None)
        torch.cuda.synchronize()
        cols = _cols(i, seed=i)
        g = _ref_cols(x, packed, s, z, cols, k).astype(np.float32)
        u = _ref_cols(x, packed, s, z, cols + i, k).astype(np.float32)
        sg = (g / (1.0 + np.exp(-g))).astype(np.float16).astype(np.float32)
        ref = (sg * u).astype(np.float16)
        assert _rel(_np(act)[:, cols], ref) <= 1e-3
        return
    g_ = torch.Generator(device=DEV).manual_seed(i + k)
    w = (torch.randn(2 * i, k, generator=g_, device=DEV) * 0.02).bfloat16()
    packed, s, z, _ = ops.w4_quantize_awq(w, 128, True, return_deq=False)
    del w
    x = torch.randn(m, k, generator=torch.Generator(device=DEV).manual_seed(9), device=DEV).bfloat16()
    act = ops.w4a16_gemm_swiglu(x, packed, s, z, 128, None)
    torch.cuda.synchronize()
    assert act.dtype == torch.bfloat16
    cols = _cols(i, seed=i)
    bits = lambda t: _np(t.view(torch.int16)).view(np.uint16)  # noqa: E731

    def half(c):
        idx = torch.as_tensor(c, device=DEV)
        deq = O.dequant_w4_bf16(_np(packed[idx]), bits(s[idx]), bits(z[idx]), k, 128)
        return O.bf16_bits_to_f32(O.w4a16_linear(bits(x), deq, None, dtype="bf16"))

    g, u = half(cols), half(cols + i)
    sg = O.bf16_bits_to_f32(O.f32_to_bf16_bits((g / (1.0 + np.exp(-g))).astype(np.float32)))
    ref = O.bf16_bits_to_f32(O.f32_to_bf16_bits((sg * u).astype(np.float32)))
    assert _rel(_np(act.float())[:, cols], ref) <= 1e-3


@pytest.mark.parametrize("dt", ["fp16", "bf16"])
def test_moe_fake_rule_mixtral_shape_sampled(dt):
    """Config 4 at full size with the module's default (fake) rule: ``SmoothQuantPackedMoeExperts``
    over T = 512 tokens, H = 4096, I = 14336, E = 8, top-2 (``fake_quant.py:124-191``).  All 512
    tokens run through the GPU chain (expert groups of their real size); 32 sampled tokens are
    recomputed by ``oracle.moe_fake``, whose per-token forward needs only those rows.  The fake-
    quant weights it uses are the module's codes times scales, after 64 sampled rows of each
    expert's codes and scales are checked bit-exact against the oracle's quantizer.  Bar: rel.
    Frobenius error <= 1e-3 over the sampled tokens."""
    _say("moe fake mixtral shape", dt)
    from mindpipe_amd.smoothquant import SmoothQuantPackedMoeExperts
    t, h, inter, e = 512, 4096, 14336, 8
    tdt = torch.float16 if dt == "fp16" else torch.bfloat16
    gen = torch.Generator(device=DEV).manual_seed(1)
    gu = (torch.randn(e, 2 * inter, h, generator=gen, device=DEV) * 0.02).to(tdt)
    dn = (torch.randn(e, h, inter, generator=gen, device=DEV) * 0.02).to(tdt)
    mod = SmoothQuantPackedMoeExperts(gu, dn, torch.nn.SiLU())
    x = torch.randn(t, h, generator=torch.Generator(device=DEV).manual_seed(0), device=DEV)
    x[:, torch.randperm(h, generator=torch.Generator().manual_seed(2))[:41].to(DEV)] *= 20
    x = x.to(tdt)
    logits = torch.randn(t, e, generator=torch.Generator().manual_seed(3)).numpy()
    ids, tw = O.mixtral_router(logits, 2)
    y = mod(x, torch.from_numpy(ids).to(DEV), torch.from_numpy(tw).to(DEV))
    torch.cuda.synchronize()
    bits = (lambda a: _np(a)) if dt == "fp16" else (lambda a: _np(a.view(torch.int16)).view(np.uint16))
    rng = np.random.default_rng(5)
    gq, dq = mod.dequantized_weights()
    val = (lambda b: b.astype(np.float32)) if dt == "fp16" else O.bf16_bits_to_f32
    for ex in range(e):   # the construction step on sampled rows: fake-quant weights exact
        for w, wq in ((gu[ex], gq[ex]), (dn[ex], dq[ex])):
            rows = torch.as_tensor(np.sort(rng.choice(w.shape[0], 64, replace=False)), device=DEV)
            _, _, rfake = O.quantize_weight_per_channel_fake(bits(w[rows]), 8, dt)
            # equal values (q * s gives +0 where the reference's round(w / s) * s gives -0)
            assert np.array_equal(val(bits(wq[rows])), val(rfake))
    toks = np.sort(rng.choice(t, 32, replace=False))
    ref = O.moe_fake(bits(x[torch.as_tensor(toks, device=DEV)]), ids[toks], tw[toks], bits(gq), bits(dq), dt,
                     prequantized=True)
    rv = ref.astype(np.float32) if dt == "fp16" else O.bf16_bits_to_f32(ref)
    err = _rel(_np(y.float())[toks], rv)
    assert err <= 1e-3, err


# the one-row VALU GEMV off the 2048 / 4096 K of the matrix-core GEMV: row counts that leave a partial
# row group (of 4, or of 8 at N >= 16384), a K that leaves a partial 2048-wide chunk, AWQ zeros and the
# symmetric export, with and without bias
ROW_GEMV_EDGES = [(8195, 8192, True, True), (6000, 11008, False, False), (16389, 8192, True, False),
                  (4099, 16384, False, True)]


@pytest.mark.parametrize("n,k,zp,with_bias", ROW_GEMV_EDGES)
def test_w4a16_one_row_gemv_edges(n, k, zp, with_bias):
    _say("w4a16 one-row gemv", n, k, zp, with_bias)
    ops = _ops()
    packed, s, z = _quant_gpu(n, k, seed=n + k, zp=zp)
    x = _x(1, k, seed=13)
    bias = (torch.randn(n, generator=torch.Generator(device=DEV).manual_seed(3), device=DEV) * 0.1).half() \
        if with_bias else None
    y = ops.w4a16_gemm(x, packed, s, z, 128, bias)
    torch.cuda.synchronize()
    cols = _cols(n, seed=n)
    assert _rel(_np(y)[:, cols], _ref_cols(x, packed, s, z, cols, k, bias)) <= 1e-3
    # every output row, against the same kernel run twice (no state left between launches)
    y2 = ops.w4a16_gemm(x, packed, s, z, 128, bias)
    assert torch.equal(y, y2)


# Edges of the one-row VALU GEMV at 34 MB layers (its 8-row, two-wave form from N = 16384): row groups
# that do not divide N (the last group clamps its rows), a partial last K chunk (K = 11008: 5.375
# chunks of 2048; K = 30720: 15 chunks), long K (16384), no zero points, a bias, and the SwiGLU form
# with an odd intermediate width.
GEMV_LARGE_EDGES = [(8200, 8192, True, True), (6104, 11008, True, False), (16400, 4096, False, True),
                (2200, 30720, True, True), (4100, 16384, False, False)]


@pytest.mark.parametrize("n,k,zp,bias", GEMV_LARGE_EDGES)
def test_w4a16_gemv_large_edges(n, k, zp, bias):
    _say("w4a16 gemv large edges", n, k, zp, bias)
    ops = _ops()
    packed, s, z = _quant_gpu(n, k, seed=n + k, zp=zp)
    x = _x(1, k, seed=13)
    b = (torch.randn(n, generator=torch.Generator(device=DEV).manual_seed(4), device=DEV) * 0.1).half() \
        if bias else None
    y = ops.w4a16_gemm(x, packed, s, z, 128, b)
    y2 = ops.w4a16_gemm(x, packed, s, z, 128, b)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)  # fixed summation order: the same bits on every call
    cols = _cols(n, seed=n, count=96)
    assert _rel(_np(y)[:, cols], _ref_cols(x, packed, s, z, cols, k, b)) <= 1e-3


@pytest.mark.parametrize("i,k,bias", [(8197, 4096, True), (4100, 8192, False)])
def test_w4a16_gemv_large_swiglu_edges(i, k, bias):
    _say("w4a16 gemv large swiglu edges", i, k, bias)
    ops = _ops()
    packed, s, z = _quant_gpu(2 * i, k, seed=i + k, zp=True)
    x = _x(1, k, seed=17)
    b = (torch.randn(2 * i, generator=torch.Generator(device=DEV).manual_seed(5), device=DEV) * 0.1).half() \
        if bias else None
    act = ops.w4a16_gemm_swiglu(x, packed, s, z, 128, b)
    torch.cuda.synchronize()
    cols = _cols(i, seed=i, count=96)
    g = _ref_cols(x, packed, s, z, cols, k, b).astype(np.float32)
    u = _ref_cols(x, packed, s, z, cols + i, k, b).astype(np.float32)
    sg = (g / (1.0 + np.exp(-g))).astype(np.float16).astype(np.float32)
    ref = (sg * u).astype(np.float16)
    assert _rel(_np(act)[:, cols], ref) <= 1e-3
