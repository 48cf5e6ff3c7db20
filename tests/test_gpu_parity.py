"""GPU parity: every HIP entry point against the numpy oracle on the same seeded inputs.

Bars (written in each test): integer codes, scales, zeros and packed words are
bit-exact; the W8A8 epilogue is bit-exact because the oracle fixes the same
float operation order; fp16 GEMM outputs have relative Frobenius error
<= 1e-3 against the oracle's dequant -> matmul.
"""
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import quant as O

pytestmark = pytest.mark.gpu
GOLD = np.load(Path(__file__).parent / "golden" / "reference_vectors.npz")
EXT = np.load(Path(__file__).parent / "golden" / "reference_ext_vectors.npz")
DEV = "cuda:0"


def _ops():
    from mindpipe_amd import ops
    return ops


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _t(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.to(DEV)


def _np(t):
    return t.detach().cpu().numpy()


def _rel(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-30))


def _w(n, k, seed=1, std=0.02):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n, k, generator=g) * std).half().numpy()


def _x(m, k, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(m, k, generator=g).half().numpy()


# ------------------------------------------------------------------ W4 quantizers
@pytest.mark.parametrize("shape,g,zp", [((48, 512), 128, True), ((8, 200), 128, True), ((48, 512), 128, False),
                                        ((64, 1024), 64, True), ((33, 4096), 128, True)])
def test_awq_quantize_bitexact(shape, g, zp):
    _say("awq_quantize", shape, g, zp)
    if shape == (48, 512):
        w = GOLD["awq_w"]
    elif shape == (8, 200):
        w = GOLD["awq_w_row"]
    else:
        w = _w(*shape, seed=7)
    packed, s, z, deq = _ops().w4_quantize_awq(_t(w), g, zp)
    rdeq, rs, rz, codes = O.pseudo_quantize_tensor(w, 4, zp, g)
    assert np.array_equal(_np(deq).view(np.uint16), rdeq.view(np.uint16))
    assert np.array_equal(_np(s).view(np.uint16), rs.view(np.uint16))
    if zp:
        assert np.array_equal(_np(z).view(np.uint16), rz.view(np.uint16))
        assert np.array_equal(_np(packed), O.pack_uint4(codes))
    else:
        assert np.array_equal(_np(packed), O.pack_int4_signed(codes))
    if shape == (48, 512) and zp:   # the reference's own outputs
        assert np.array_equal(_np(deq).view(np.uint16), GOLD["awq_deq"].view(np.uint16))
        assert np.array_equal(_np(z).view(np.uint16), GOLD["awq_z"].view(np.uint16))


def test_gptq_rtn_bitexact():
    _say("gptq_rtn")
    w = GOLD["gptq_w"]
    iw, packed, s = _ops().w4_quantize_gptq_rtn(_t(w.astype(np.float32)), 128)
    assert np.array_equal(_np(iw), GOLD["gptq_int"])
    assert np.array_equal(_np(s).view(np.uint16), GOLD["gptq_scale"].view(np.uint16))
    assert np.array_equal(_np(packed), O.pack_int4_signed(GOLD["gptq_int"]))


def test_pack_int4_kats_and_random():
    _say("pack_int4")
    ops = _ops()
    vals = np.array([[-8, -7, -1, 0, 1, 6, 7, -3, 4, 2]], np.int8)
    p = ops.pack_int4(_t(vals))
    assert _np(p).tolist() == [[1609139984, 172]]
    assert np.array_equal(_np(ops.unpack_int4(p, 10)), vals)
    iw = np.array([[-8, -7, -1, 0, 1, 6, 7, -3], [7, 6, 1, 0, -1, -7, -8, 3]], np.int8)
    assert _np(ops.pack_int4(_t(iw))).tolist() == [[1609139984], [-1340634641]]
    assert np.array_equal(_np(ops.pack_int4(_t(GOLD["pack_in"]))), GOLD["pack_out"])
    with pytest.raises(ValueError):
        ops.pack_int4(_t(np.array([[9, 0]], np.int8)))


# ------------------------------------------------------------------ W4A16 GEMM
W4_CASES = [(1, 4096, 4096), (16, 4096, 4096), (3, 512, 1024), (17, 256, 2048), (33, 384, 1024), (64, 128, 512),
            (65, 256, 512), (200, 320, 1024), (256, 4096, 4096),
            # batched small-M kernel: 17..32 rows with 4 column tiles per wave, 8 split waves, tail columns
            (24, 8192, 1024), (32, 1024, 2048), (40, 400, 1024), (12, 20480, 512),
            # four column tiles from N = 10240 up to 16 rows (the 70B q/k/v), ragged last tile
            (16, 10240, 1024), (12, 10300, 512),
            # one-row GEMV: partial 2048-wide K chunk, N not a multiple of the rows per wave, odd chunk count
            (1, 37, 768), (1, 301, 2304), (1, 1001, 11008), (1, 64, 6144),
            # one-row matrix-core GEMV (K = 2048, 4096): N not a multiple of its 16-row tiles
            (1, 2048, 2048), (1, 1000, 4096), (1, 24, 2048), (1, 4097, 4096), (1, 8, 2048),
            # 2..8 rows (four-row MFMA kernel): half-filled last K chunk, N not a multiple of 16, split-K waves
            (2, 4096, 4096), (4, 1000, 2304), (5, 4096, 11008), (8, 12288, 4096), (7, 300, 1280), (6, 72, 512),
            # 33..64 rows: one 64-row tile where N <= 8192 (fp16), else two 32-row parts of one grid
            # (padding workgroups, 4 / 2 / 1 column tiles)
            (48, 12288, 4096), (64, 8192, 2048), (37, 1000, 1024), (57, 4096, 1280),
            # 65..512 rows where the prefill grid would fill at most half the CUs: batched kernel in 32-row
            # parts (up to 12), ragged last part
            (96, 4096, 4096), (384, 1024, 2048), (130, 520, 1024),
            # prefill tiles: ragged rows and columns; mid-M with a large grid (N = 12288, 24000)
            (600, 1000, 1024), (2048, 384, 512), (300, 12288, 1024), (129, 24000, 512)]


@pytest.mark.parametrize("m,n,k", W4_CASES)
@pytest.mark.parametrize("zp", [True, False])
def test_w4a16_gemm_matches_dequant_matmul(m, n, k, zp):
    _say("w4a16", m, n, k, zp)
    w = _w(n, k, seed=1)
    x = _x(m, k, seed=0)
    if zp:
        rdeq, rs, rz, codes = O.pseudo_quantize_tensor(w, 4, True, 128)
        packed = O.pack_uint4(codes)
    else:
        iw, rs, _ = O.gptq_rtn_quantize(w.astype(np.float32), 4, 128)
        packed = O.pack_int4_signed(iw)
        rz = None
        rdeq = O.dequant_w4_fp16(packed, rs, None, k, 128)
    bias = (np.random.default_rng(5).standard_normal(n) * 0.1).astype(np.float16)
    ref = O.w4a16_linear(x, rdeq, bias)
    y = _ops().w4a16_gemm(_t(x), _t(packed), _t(rs), None if rz is None else _t(rz), 128, _t(bias))
    err = _rel(_np(y), ref)
    assert err <= 1e-3, err   # bar: ||Y - Y_ref||_F / ||Y_ref||_F <= 1e-3


@pytest.mark.parametrize("m,i,k", [(1, 2048, 4096), (1, 1001, 2304), (1, 300, 11008), (8, 2048, 4096), (16, 1000, 1024),
                                   (24, 4096, 512), (40, 520, 2048), (64, 256, 1024), (3, 1001, 2304),
                                   (6, 300, 11008), (64, 8192, 2048), (45, 1000, 1024), (8, 16400, 512),
                                   # above 64 rows: the batched kernel's SwiGLU form in row parts, and the
                                   # prefill kernel's (128- and 256-row tiles) where w4a16_gemm takes it
                                   (100, 1000, 1024), (300, 520, 512), (65, 64, 256), (130, 8200, 256),
                                   (520, 300, 512)])
@pytest.mark.parametrize("zp", [True, False])
def test_w4a16_gemm_swiglu_matches_two_step(m, i, k, zp):
    """Fused gate/up GEMM + SiLU-mul against silu_mul(w4a16_gemm) (bit-exact where both run the
    one-row VALU GEMV, whose per-row arithmetic is the same; <= 1 ulp for the batched kernel, whose K
    split may differ; rel. <= 1e-3 where w4a16_gemm takes the one-row matrix-core GEMV, K = 2048 /
    4096, or, above 64 rows, a different kernel than the fused form's prefill kernel) and against the
    oracle's dequant -> matmul -> SiLU-mul (rel. error <= 1e-3)."""
    _say("w4a16 swiglu", m, i, k, zp)
    ops = _ops()
    n2 = 2 * i
    w = _w(n2, k, seed=3)
    x = _x(m, k, seed=4)
    if zp:
        rdeq, rs, rz, codes = O.pseudo_quantize_tensor(w, 4, True, 128)
        packed = O.pack_uint4(codes)
    else:
        iw, rs, _ = O.gptq_rtn_quantize(w.astype(np.float32), 4, 128)
        packed = O.pack_int4_signed(iw)
        rz = None
        rdeq = O.dequant_w4_fp16(packed, rs, None, k, 128)
    bias = (np.random.default_rng(6).standard_normal(n2) * 0.1).astype(np.float16)
    args = (_t(packed), _t(rs), None if rz is None else _t(rz), 128, _t(bias))
    act = ops.w4a16_gemm_swiglu(_t(x), *args)
    two = ops.silu_mul(ops.w4a16_gemm(_t(x), *args))
    d = (act.view(torch.int16).int() - two.view(torch.int16).int()).abs()
    if m == 1 and k in (2048, 4096):
        assert _rel(_np(act), _np(two)) <= 1e-3
    elif m == 1:
        assert torch.equal(act, two)
    elif m > 64:  # the prefill kernel's SwiGLU form; w4a16_gemm may take the batched kernel there
        assert _rel(_np(act), _np(two)) <= 1e-3
    else:
        assert int(d.max()) <= 1 and float((d == 0).float().mean()) >= 0.99
    gu = O.w4a16_linear(x, rdeq, bias).astype(np.float32)
    g, u = gu[:, :i], gu[:, i:]
    ref = (g / (1.0 + np.exp(-g))) * u
    assert _rel(_np(act).astype(np.float32), ref) <= 1e-3   # bar: ||act - ref||_F / ||ref||_F <= 1e-3


@pytest.mark.parametrize("m,i,k", [(1, 2048, 4096), (1, 300, 11008), (8, 2048, 4096), (16, 1000, 1024),
                                   (40, 520, 2048), (64, 256, 1024), (3, 1001, 2304), (100, 300, 1024),
                                   (12, 16400, 512), (300, 520, 512), (520, 300, 512)])
@pytest.mark.parametrize("zp", [True, False])
def test_w4a16_gemm_swiglu_bf16_matches_oracle(m, i, k, zp):
    """bf16 fused gate/up GEMM + SiLU-mul (the batched kernel's bf16 SwiGLU form for M <= 64, the bf16
    GEMM then silu_mul above) against the oracle: gate and up = F.linear on the bf16 pseudo-quantized
    weight, each rounded to bf16, then round(round(silu(gate)) * up) in bf16; rel. error <= 1e-3.
    Against silu_mul(w4a16_gemm) in bf16: <= 1 bf16 ulp (their K splits differ), >= 99% equal."""
    _say("w4a16 swiglu bf16", m, i, k, zp)
    ops = _ops()
    n2 = 2 * i
    rng = np.random.default_rng(m + i + k)
    w = O.f32_to_bf16_bits((rng.standard_normal((n2, k)) * 0.02).astype(np.float32))
    x = O.f32_to_bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    bias = O.f32_to_bf16_bits((rng.standard_normal(n2) * 0.1).astype(np.float32))
    rdeq, rs, rz, codes = O.pseudo_quantize_tensor(w, 4, zp, 128, dtype="bf16")
    packed = O.pack_uint4(codes) if zp else O.pack_int4_signed(codes)
    tb = lambda a: _t(a.view(np.int16), torch.bfloat16)  # noqa: E731
    args = (_t(packed), tb(rs), None if rz is None else tb(rz), 128, tb(bias))
    act = ops.w4a16_gemm_swiglu(tb(x), *args)
    assert act.dtype == torch.bfloat16 and act.shape == (m, i)
    two = ops.silu_mul(ops.w4a16_gemm(tb(x), *args))
    d = (act.view(torch.int16).int() - two.view(torch.int16).int()).abs()
    if m > 64:  # the prefill kernel's SwiGLU form; w4a16_gemm may take the batched kernel there
        assert _rel(_np(act.float()), _np(two.float())) <= 1e-3
    else:
        assert int(d.max()) <= 1 and float((d == 0).float().mean()) >= 0.99
    gu = O.bf16_bits_to_f32(O.w4a16_linear(x, rdeq, bias, dtype="bf16"))
    g, u = gu[:, :i], gu[:, i:]
    rb = lambda v: O.bf16_bits_to_f32(O.f32_to_bf16_bits(v.astype(np.float32)))  # noqa: E731
    ref = rb(rb(g / (np.float32(1.0) + np.exp(-g))) * u)
    assert _rel(_np(act.float()), ref) <= 1e-3   # bar: ||act - ref||_F / ||ref||_F <= 1e-3


def test_awq_quantize_bf16_matches_reference():
    """AWQ pseudo_quantize_tensor in bf16 arithmetic (asym with a constant group; sym): the
    dequantized weight, scales and zeros bit-exact to the reference's bf16 outputs."""
    _say("awq bf16")
    w = EXT["awqb_w"].view(np.uint16)
    wt = torch.from_numpy(EXT["awqb_w"]).view(torch.bfloat16).to(DEV)
    packed, s, z, deq = _ops().w4_quantize_awq(wt, 128, True)
    bits = lambda t: _np(t.view(torch.int16)).view(np.uint16)  # noqa: E731
    assert np.array_equal(bits(deq), EXT["awqb_deq"].view(np.uint16))
    assert np.array_equal(bits(s), EXT["awqb_s"].view(np.uint16))
    assert np.array_equal(bits(z), EXT["awqb_z"].view(np.uint16))
    _, _, _, codes = O.pseudo_quantize_tensor(w, 4, True, 128, dtype="bf16")
    assert np.array_equal(_np(packed), O.pack_uint4(codes))
    _, _, _, deq_s = _ops().w4_quantize_awq(wt, 128, False)
    assert np.array_equal(bits(deq_s), EXT["awqb_sym_deq"].view(np.uint16))


# bf16: (m, n, k).  1 to 16 rows with K % 128 == 0: the matrix-core small-M kernel -- one row and
# several, ragged N, one to sixteen waves per row block, odd group counts (K = 640: five groups, a
# round with one group; K = 11008: 86 groups over sixteen waves, the last one idle) and a long K
# (K = 30720: 240 groups; K = 36864 / 40064: 18 / 20 groups per wave, so the prologue's first batch is
# full and a second one follows, and the last wave of K = 40064 has 13).  2 to 64 rows with K % 256 == 0
# and an even group count: the batched kernel's bf16 form (16- and 32-row parts, one to four column
# tiles per wave, ragged N, 86 groups); other K with up to 16 rows (640, 1152, 40064) stay on the small-M
# kernel.  65 to 512 rows where the prefill grid is small (130 / 200 rows): the batched form in parts.
# Above that, with K % 64 == 0 and a group of 32 or 128: the prefill kernel's bf16 form (128- and 256-row
# tiles, ragged M / N).  One row past its LDS bound (K = 40960) and the other shapes: the
# dequantising MFMA GEMM (tiled) and its any-K kernel (K = 96).
W4_BF16_CASES = [(1, 4096, 4096), (16, 4096, 4096), (3, 1000, 1024), (1, 17, 128), (7, 33, 640),
                 (1, 4096, 11008), (12, 300, 2048), (16, 520, 11008), (9, 2048, 8192), (1, 2050, 2048),
                 (1, 300, 30720), (4, 64, 30720), (1, 37, 36864), (2, 100, 40064), (1, 48, 40960),
                 (24, 4096, 4096), (33, 12288, 4096), (40, 520, 2048), (48, 4096, 11008), (64, 8200, 1024),
                 (16, 300, 1152), (2, 22016, 4096), (130, 1000, 1024), (80, 130, 320), (700, 520, 2048),
                 (17, 96, 512), (64, 384, 512), (200, 320, 1024), (300, 12288, 4096), (5, 256, 8192),
                 (2, 100, 96)]


@pytest.mark.parametrize("m,n,k", W4_BF16_CASES)
@pytest.mark.parametrize("zp", [True, False])
def test_w4a16_gemm_bf16_matches_dequant_matmul(m, n, k, zp):
    """bf16 W4A16 against F.linear(x, pseudo_quantize_tensor(w)) in bf16 (fp32 accumulation, one
    rounding): rel. Frobenius error <= 1e-3."""
    _say("w4a16 bf16", m, n, k, zp)
    g = 128 if k % 128 == 0 else 32
    rng = np.random.default_rng(m + n + k)
    w = O.f32_to_bf16_bits((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = O.f32_to_bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    bias = O.f32_to_bf16_bits((rng.standard_normal(n) * 0.1).astype(np.float32))
    rdeq, rs, rz, codes = O.pseudo_quantize_tensor(w, 4, zp, g, dtype="bf16")
    packed = O.pack_uint4(codes) if zp else O.pack_int4_signed(codes)
    ref = O.bf16_bits_to_f32(O.w4a16_linear(x, rdeq, bias, dtype="bf16"))
    tb = lambda a: _t(a.view(np.int16), torch.bfloat16)  # noqa: E731
    y = _ops().w4a16_gemm(tb(x), _t(packed), tb(rs), None if rz is None else tb(rz), g, tb(bias))
    assert y.dtype == torch.bfloat16
    err = _rel(_np(y.float()), ref)
    assert err <= 1e-3, err   # bar: ||Y - Y_ref||_F / ||Y_ref||_F <= 1e-3


def test_w4a16_odd_shapes_use_exact_path():
    _say("w4a16 odd")
    # export KAT: K = 8, g = 4 (tests/test_vllm_real_quant_export.py:105-152)
    iw = np.array([[-8, -7, -1, 0, 1, 6, 7, -3], [7, 6, 1, 0, -1, -7, -8, 3]], np.int8)
    scale = np.array([[0.1, 0.2], [0.3, 0.4]], np.float16)
    packed = O.pack_int4_signed(iw)
    x = _x(5, 8, seed=3)
    deq = O.dequant_w4_fp16(packed, scale, None, 8, 4)
    ref = O.w4a16_linear(x, deq)
    y = _ops().w4a16_gemm(_t(x), _t(packed), _t(scale), None, 4, None)
    assert _rel(_np(y), ref) <= 1e-3


def test_w4a16_empty_batch():
    w = _w(64, 256)
    _, rs, rz, codes = O.pseudo_quantize_tensor(w, 4, True, 128)
    y = _ops().w4a16_gemm(torch.empty((0, 256), dtype=torch.float16, device=DEV), _t(O.pack_uint4(codes)),
                          _t(rs), _t(rz), 128, None)
    assert y.shape == (0, 64)


# ------------------------------------------------------------------ W8 quantizers
# k: 16-byte kernel (k a multiple of the values per 16 bytes), scalar kernel (4099), a short row
@pytest.mark.parametrize("k", [4096, 4099, 24])
@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
def test_per_token_quant_fp32_rule_bitexact(dtype, k):
    _say("per_token fp32 rule", dtype, k)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(67, k, generator=g)
    x[:, torch.randperm(k, generator=g)[:41]] *= 20
    x[5] = 0.0
    x[6] = (torch.arange(k) - k // 2) * 0.5
    tdt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[dtype]
    xt = x.to(tdt)
    q, s = _ops().quant_per_token_i8(xt.to(DEV))
    xn = xt.view(torch.int16).numpy().view(np.uint16) if dtype == "bf16" else xt.numpy()
    rq, rs = O.quantize_per_token_runtime(xn, in_dtype=dtype)
    assert np.array_equal(_np(q), rq)
    assert np.array_equal(_np(s), rs)


def test_per_token_quant_fp16_rule_matches_reference():
    _say("per_token fp16 rule")
    x = GOLD["sq_x"]
    q, s = _ops().quant_per_token_i8(_t(x), True)
    rq, rs, rfake = O.quantize_activation_per_token_fake(x)
    assert np.array_equal(_np(q), rq)
    assert np.array_equal(_np(s).view(np.uint16), rs.view(np.uint16))
    # int8 codes cannot carry the sign of a zero, so compare values (-0.0 == 0.0)
    fake = (_np(q).astype(np.float32) * _np(s).astype(np.float32)[:, None]).astype(np.float16)
    assert np.array_equal(fake, GOLD["sq_x_fq"])


def _fake_values(q, s, dt):
    """Values ``q * s`` of stored codes rounded to the rule's dtype, as float32 (int8 codes carry
    no sign of zero, so values are compared, -0.0 == 0.0)."""
    v = q.float() * s.float().unsqueeze(-1)
    return _np((v.bfloat16() if dt == "bf16" else v.half()).float())


def _both_128_rows(codes):
    """Rows whose fake-rule codes reach both +128 and -128 (stored with +128 clamped to 127)."""
    c = codes.astype(np.int32)
    return (c >= 128).any(-1) & (c <= -128).any(-1)


@pytest.mark.parametrize("which", ["act", "weight"])
def test_fake_rule_bf16_matches_reference(which):
    """bf16 fake rule (quantize_*_absmax in bf16): q * s equals the reference's fake values on
    every row (rows reaching +128 are stored negated); the codes are the oracle's codes up to
    that sign, within [-128, 127]."""
    _say("fake rule bf16", which)
    ops = _ops()
    xb = EXT["sqb_x" if which == "act" else "sqb_w"]
    ref = EXT["sqb_x_fq" if which == "act" else "sqb_w_fq"].view(np.uint16)
    xt = torch.from_numpy(xb).view(torch.bfloat16).to(DEV)
    if which == "act":
        q, s = ops.quant_per_token_i8(xt, True)
        assert s.dtype == torch.bfloat16
    else:
        q, s32, s = ops.w8_quantize_per_channel(xt, "fake")
        assert torch.equal(s32, s.float())
    codes, _, _ = O.quantize_activation_per_token_fake(xb.view(np.uint16), 8, "bf16")
    assert not _both_128_rows(codes).any()
    assert np.array_equal(_fake_values(q, s, "bf16"), O.bf16_bits_to_f32(ref))
    sign = np.where(_np(s.float()) < 0, -1, 1)[:, None]
    assert np.array_equal(_np(q).astype(np.int32) * sign, codes.astype(np.int32))


def test_fake_rule_bf16_random_rows_and_ties():
    """bf16 fake rule on 2000 random rows with outliers plus +-a rows (every code +-128):
    bit-exact fake values except on rows reaching both +-128, where only the +128 entries move
    by one code."""
    _say("fake rule bf16 random")
    g = torch.Generator().manual_seed(9)
    x = torch.randn(2000, 1024, generator=g)
    x[:, torch.randperm(1024, generator=g)[:10]] *= 20
    x[0] = torch.tensor([3.0, -3.0]).repeat(512)
    x[1] = 1.0
    xb = x.bfloat16()
    bits = xb.view(torch.int16).numpy().view(np.uint16)
    codes, _, fake = O.quantize_activation_per_token_fake(bits, 8, "bf16")
    q, s = _ops().quant_per_token_i8(xb.to(DEV), True)
    got = _fake_values(q, s, "bf16")
    both = _both_128_rows(codes)
    assert np.array_equal(got[~both], O.bf16_bits_to_f32(fake)[~both])
    qn = _np(q).astype(np.int32)
    assert qn.min() >= -128 and qn.max() <= 127
    for r in np.nonzero(both)[0]:
        d = codes[r].astype(np.int32) - qn[r]
        assert set(np.unique(d)) <= {0, 1} and np.all((d == 0) | (codes[r] == 128))


def test_w8_quantize_export_and_fake_rules():
    _say("w8 quantize")
    ops = _ops()
    q, s32, s16 = ops.w8_quantize_per_channel(_t(GOLD["sq_w"]), "export")
    assert np.array_equal(_np(q), GOLD["ex_q"])
    assert np.array_equal(_np(s16).view(np.uint16), GOLD["ex_s"][:, 0].view(np.uint16))
    wb = torch.from_numpy(GOLD["ex_wb_bits"]).view(torch.bfloat16).to(DEV)
    qb, _, sb = ops.w8_quantize_per_channel(wb, "export")
    assert np.array_equal(_np(qb), GOLD["ex_qb"])
    assert np.array_equal(_np(sb.view(torch.int16)), GOLD["ex_sb_bits"][:, 0])
    qf, sf32, sf16 = ops.w8_quantize_per_channel(_t(GOLD["sq_w"]), "fake")
    fake = (_np(qf).astype(np.float32) * _np(sf32)[:, None]).astype(np.float16)
    assert np.array_equal(fake, GOLD["sq_w_fq"])   # values; int8 codes drop the sign of zero
    for case in [{"w": [[-1, 0, 1], [2, 3, 4]], "q": [[-127, 0, 127], [64, 95, 127]]},
                 {"w": [[-2, -1, 0], [1, 2, 3]], "q": [[-127, -64, 0], [42, 85, 127]]}]:
        qk, _, _ = ops.w8_quantize_per_channel(_t(np.array(case["w"], np.float16)), "export")
        assert _np(qk).tolist() == case["q"]
    with pytest.raises(ValueError):
        ops.w8_quantize_per_channel(_t(np.array([[1.0, np.inf]], np.float16)), "export")


# ------------------------------------------------------------------ W8A8 GEMM
W8_CASES = [(1, 11008, 4096), (16, 11008, 4096), (5, 1000, 256), (17, 512, 1024), (64, 384, 512), (65, 256, 512),
            (256, 1000, 1024), (300, 384, 4096), (7, 100, 48), (1100, 300, 256), (2048, 520, 320),
            # large-M kernel: four register stages over 3 loop trips, two stages (K % 256 != 0)
            (1024, 640, 768), (1300, 700, 384),
            # large-M kernel with odd N: the unpaired store path
            (1024, 333, 256),
            # large-M kernel: twenty loop trips, partial row and column tiles
            (1100, 600, 2560),
            # row-contiguous GEMV (M <= 2): K past the last 1 KB chunk, M = 2, tiny K, K = 11008
            (2, 300, 1040), (1, 257, 4112), (2, 64, 16), (1, 100, 11008),
            # skinny kernel where the whole K fits the 76 KB LDS budget but not the staging
            # registers (more than 4096 sixteen-byte pieces): K split into chunks
            (17, 512, 4096), (18, 300, 4096), (7, 256, 11008), (5, 256, 14336), (33, 256, 2048),
            # C2 sweep at M = 256 (mid-M direct-to-LDS kernel) on the full N x K
            (256, 11008, 4096),
            # mid-M kernel (64 .. 256 tiles of 128 x 128): partial row and column tiles, K of 1 to 9
            # steps of 128 (partial four-step loop groups), odd N (the unpaired store path)
            (200, 8200, 512), (65, 8320, 1152), (384, 2700, 640), (1000, 2048, 128), (129, 12001, 256),
            # direct-to-LDS skinny kernel (3..32 rows, 1 to 4 column tiles per workgroup): two 16-row
            # tiles, waves with one and two K steps, odd N, partial column tiles
            (32, 2000, 640), (3, 5000, 512), (24, 16000, 1024), (13, 12001, 768),
            # tiled kernel: the LDS-staged 16-byte-store epilogue with partial row and column tiles
            # (N % 8 == 0), and the two-byte-store epilogue (N % 8 != 0)
            (200, 1000, 512), (100, 333, 512),
            # 33..64 rows: the tiled kernel where its grid is large (N = 11008), the skinny kernel where
            # it is small (N = 4096)
            (48, 11008, 4096), (64, 11008, 1024), (40, 4096, 1024)]


@pytest.mark.parametrize("m,n,k", W8_CASES)
@pytest.mark.parametrize("out", ["fp16", "bf16", "fp32"])
def test_w8a8_gemm_bitexact(m, n, k, out):
    _say("w8a8", m, n, k, out)
    rng = np.random.default_rng(m * 7 + n)
    qx = rng.integers(-127, 128, (m, k)).astype(np.int8)
    qw = rng.integers(-127, 128, (n, k)).astype(np.int8)
    sx = (rng.random(m) * 0.01).astype(np.float32)
    sw = (rng.random(n) * 0.001).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.1).astype(np.float16)
    odt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[out]
    y = _ops().w8a8_gemm(_t(qx), _t(sx), _t(qw), _t(sw), _t(bias), odt)
    ref = O.w8a8_linear_runtime(qx, sx, qw, sw, bias, out_dtype=out)
    if out == "fp32":
        assert np.array_equal(_np(y).view(np.uint32), ref.view(np.uint32))   # bar: bit-exact
        return
    got = _np(y.view(torch.int16)).view(np.uint16) if out == "bf16" else _np(y).view(np.uint16)
    assert np.array_equal(got, ref.view(np.uint16))   # bar: bit-exact


def _random_w8_shapes(count=40, seed=11):
    """Seeded shapes across every W8A8 routing range: rows 1..1100, N 1..13000 (odd included), K a
    multiple of 16, 64 or 128 from 16 to 4608."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        m = int(rng.choice([1, 2, 3, 5, 8, 13, 16, 17, 24, 31, 32, 33, 48, 64, 65, 97, 128, 200, 256, 300, 511, 1100]))
        n = int(rng.integers(1, 13000))
        k = int(rng.choice([16, 64, 128])) * int(rng.integers(1, 37))
        if m * n * k <= 6e9:
            out.append((m, n, k))
    return out


@pytest.mark.parametrize("m,n,k", _random_w8_shapes())
def test_w8a8_gemm_random_shapes(m, n, k):
    """Seeded shapes over every routing range of mp_w8a8_gemm (GEMV, both skinny kernels, tiled, mid-M,
    large-M, the any-shape fallback): fp16 output bit-exact against the oracle."""
    _say("w8a8 random", m, n, k)
    rng = np.random.default_rng(m * 131 + n * 7 + k)
    qx = rng.integers(-127, 128, (m, k)).astype(np.int8)
    qw = rng.integers(-127, 128, (n, k)).astype(np.int8)
    sx = (rng.random(m) * 0.01).astype(np.float32)
    sw = (rng.random(n) * 0.001).astype(np.float32)
    y = _ops().w8a8_gemm(_t(qx), _t(sx), _t(qw), _t(sw), None, torch.float16)
    ref = O.w8a8_linear_runtime(qx, sx, qw, sw, None, out_dtype="fp16")
    assert np.array_equal(_np(y).view(np.uint16), ref.view(np.uint16))   # bar: bit-exact


def test_w8a8_gemm_large_rows_subset():
    """M = 4096, N = 11008, K = 4096 (BASELINE config): bit-exact on 96 sampled rows x all columns."""
    _say("w8a8 full size")
    m, n, k = 4096, 11008, 4096
    gen = torch.Generator(device=DEV).manual_seed(3)
    qx = torch.randint(-127, 128, (m, k), generator=gen, device=DEV, dtype=torch.int8)
    qw = torch.randint(-127, 128, (n, k), generator=gen, device=DEV, dtype=torch.int8)
    sx = torch.rand(m, generator=gen, device=DEV) * 0.01
    sw = torch.rand(n, generator=gen, device=DEV) * 0.001
    y = _ops().w8a8_gemm(qx, sx, qw, sw, None, torch.float16)
    rows = np.random.default_rng(0).choice(m, 96, replace=False)
    rows = np.concatenate([rows, [0, 127, 128, m - 1]])
    ref = O.w8a8_linear_runtime(_np(qx)[rows], _np(sx)[rows], _np(qw), _np(sw))
    assert np.array_equal(_np(y)[rows].view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("out", ["fp16", "bf16"])
def test_w8a8_gemm_persistent_partial_tiles(out):
    """M = 4100, N = 5000, K = 512: 17 x 20 tiles of 256 x 256 over a persistent grid (more tiles than
    CUs), with a partial last row tile (4 rows) and column tile (136 columns); bit-exact on sampled
    rows (those of the partial tile included) x all columns."""
    _say("w8a8 persistent partial tiles", out)
    m, n, k = 4100, 5000, 512
    gen = torch.Generator(device=DEV).manual_seed(5)
    qx = torch.randint(-127, 128, (m, k), generator=gen, device=DEV, dtype=torch.int8)
    qw = torch.randint(-127, 128, (n, k), generator=gen, device=DEV, dtype=torch.int8)
    sx = torch.rand(m, generator=gen, device=DEV) * 0.01
    sw = torch.rand(n, generator=gen, device=DEV) * 0.001
    bias = (torch.randn(n, generator=gen, device=DEV) * 0.1).half()
    odt = torch.float16 if out == "fp16" else torch.bfloat16
    y = _ops().w8a8_gemm(qx, sx, qw, sw, bias, odt)
    rows = np.random.default_rng(1).choice(m, 64, replace=False)
    rows = np.unique(np.concatenate([rows, [0, 255, 256, 4095, 4096, 4097, 4098, 4099]]))
    ref = O.w8a8_linear_runtime(_np(qx)[rows], _np(sx)[rows], _np(qw), _np(sw), _np(bias), out_dtype=out)
    got = _np(y.view(torch.int16)).view(np.uint16) if out == "bf16" else _np(y).view(np.uint16)
    assert np.array_equal(got[rows], ref.view(np.uint16))


def test_w8a8_end_to_end_vs_fake_reference():
    """SmoothQuant linear: GPU quantizers + int8 GEMM against the reference fake-quant F.linear (fp16 rules)."""
    _say("w8a8 e2e")
    x = _x(16, 1024, seed=0)
    w = _w(512, 1024, seed=1)
    ops = _ops()
    q, s16 = ops.quant_per_token_i8(_t(x), True)
    qw, sw32, _ = ops.w8_quantize_per_channel(_t(w), "fake")
    y = ops.w8a8_gemm(q, s16.float(), qw, sw32, None, torch.float16)
    ref = O.w8a8_linear_fake(x, w)
    assert _rel(_np(y), ref) <= 1e-3


# ------------------------------------------------------------------ MoE
def _moe_case(t, h, inter, e, seed=0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((t, h)).astype(np.float16)
    ids, tw = O.mixtral_router(rng.standard_normal((t, e)).astype(np.float32), 2)
    wgu = (rng.standard_normal((e, 2 * inter, h)) * 0.02).astype(np.float16)
    wdn = (rng.standard_normal((e, h, inter)) * 0.02).astype(np.float16)
    q13 = np.stack([O.quantize_weight_per_channel_export(wgu[i])[0] for i in range(e)])
    s13 = np.stack([O.quantize_weight_per_channel_export(wgu[i])[1] for i in range(e)])
    q2 = np.stack([O.quantize_weight_per_channel_export(wdn[i])[0] for i in range(e)])
    s2 = np.stack([O.quantize_weight_per_channel_export(wdn[i])[1] for i in range(e)])
    return x, ids, tw, q13, s13, q2, s2


# (t, h, inter, e): experts of up to ~300 rows (two 256-row chunks on the grouped large-M kernel),
# an intermediate size that is not a multiple of 128 (tiled kernel), a nearly empty batch
@pytest.mark.parametrize("t,h,inter,e", [(64, 256, 512, 8), (200, 512, 384, 4), (3, 128, 128, 8),
                                         (600, 256, 256, 4), (64, 256, 320, 4), (256, 1024, 512, 8)])
def test_moe_chain_matches_oracle(t, h, inter, e):
    _say("moe", t, h, inter, e)
    x, ids, tw, q13, s13, q2, s2 = _moe_case(t, h, inter, e)
    ops = _ops()
    routed, rscale, row_of_slot, offs = ops.moe_permute_quant(_t(x), _t(ids), e)
    # routing: offsets and stable placement are exact
    counts = np.bincount(ids.reshape(-1), minlength=e)
    assert np.array_equal(_np(offs), np.concatenate([[0], np.cumsum(counts)]))
    order = np.argsort(ids.reshape(-1), kind="stable")
    exp_row = np.empty_like(order)
    exp_row[order] = np.arange(order.size)
    assert np.array_equal(_np(row_of_slot), exp_row)
    qx, sx = O.quantize_per_token_runtime(x)
    tok_of_row = order // 2
    assert np.array_equal(_np(routed), qx[tok_of_row])
    assert np.array_equal(_np(rscale), sx[tok_of_row])
    y = ops.moe_w8a8_forward(_t(x), _t(ids), _t(tw), _t(q13), _t(s13), _t(q2), _t(s2))
    ref, inter_codes = O.moe_runtime(x, ids, tw, q13, s13, q2, s2, return_intermediate=True)
    err = _rel(_np(y), ref)
    assert err <= 1e-3, err
    # requant codes: equal except where silu's exp lands on a rounding boundary
    qh, sh = ops.moe_gmm1_swiglu_quant(routed, rscale, _t(q13), _t(s13), offs, inter)
    qh = _np(qh)
    agree, total = 0, 0
    for ex, (tok, pos, rq, rs) in inter_codes.items():
        rows = exp_row[tok * 2 + pos]
        agree += np.sum(qh[rows] == rq)
        total += rq.size
        assert np.max(np.abs(qh[rows].astype(int) - rq.astype(int))) <= 1
    assert agree / total >= 0.999


def _moe_module(gu, dn, dt, rule="fake"):
    from mindpipe_amd.smoothquant import SmoothQuantPackedMoeExperts
    tdt = torch.float16 if dt == "fp16" else torch.bfloat16
    cv = (lambda a: torch.from_numpy(np.ascontiguousarray(a))) if dt == "fp16" else \
        (lambda a: torch.from_numpy(np.ascontiguousarray(a)).view(torch.bfloat16))
    return SmoothQuantPackedMoeExperts(cv(gu).to(DEV), cv(dn).to(DEV), torch.nn.SiLU(), scale_rule=rule), cv, tdt


@pytest.mark.parametrize("tag,dt", [("f16", "fp16"), ("bf16", "bf16")])
def test_moe_fake_rule_matches_reference_module(tag, dt):
    """SmoothQuantPackedMoeExperts (default fake rule) against the output the reference module
    wrote for the same weights, tokens and routing (fake_quant.py:124-191): rel. Frobenius
    error <= 1e-3 (fp32 sums in a different order, silu's exp), most elements bit-identical."""
    _say("moe fake vs reference", dt)
    mod, cv, tdt = _moe_module(EXT[f"moe_{tag}_gu"], EXT[f"moe_{tag}_dn"], dt)
    x = cv(EXT[f"moe_{tag}_x"]).to(DEV)
    ids = torch.from_numpy(EXT[f"moe_{tag}_ids"]).long().to(DEV)
    w = torch.from_numpy(EXT[f"moe_{tag}_w"]).to(DEV)
    y = mod(x, ids, w)
    assert y.dtype == tdt and y.shape == x.shape
    ref = EXT[f"moe_{tag}_y"]
    yv = _np(y.float())
    rv = ref.astype(np.float32) if dt == "fp16" else O.bf16_bits_to_f32(ref.view(np.uint16))
    err = _rel(yv, rv)
    assert err <= 1e-3, err   # bar: rel. Frobenius error <= 1e-3 against the reference module
    same = np.mean(_np(y.view(torch.int16)).view(np.uint16) == ref.view(np.uint16))
    assert same >= 0.9, same
    assert not yv[0].any()    # token 0 is all zeros in the fixture


@pytest.mark.parametrize("dt", ["fp16", "bf16"])
def test_moe_fake_rule_matches_oracle_larger(dt):
    """Fake-rule chain at T = 300, H = 1024, I = 768, E = 8 (experts over 64 rows, tiled and
    grouped kernels) against oracle.moe_fake: rel. Frobenius error <= 1e-3."""
    _say("moe fake larger", dt)
    t, h, inter, e = 300, 1024, 768, 8
    rng = np.random.default_rng(21)
    xf = rng.standard_normal((t, h)).astype(np.float32)
    xf[:, rng.choice(h, 10, replace=False)] *= 20
    ids, tw = O.mixtral_router(rng.standard_normal((t, e)).astype(np.float32), 2)
    guf = (rng.standard_normal((e, 2 * inter, h)) * 0.02).astype(np.float32)
    dnf = (rng.standard_normal((e, h, inter)) * 0.02).astype(np.float32)
    conv = (lambda a: a.astype(np.float16)) if dt == "fp16" else O.f32_to_bf16_bits
    x, gu, dn = conv(xf), conv(guf), conv(dnf)
    mod, cv, _ = _moe_module(gu, dn, dt)
    y = mod(cv(x).to(DEV), torch.from_numpy(ids).to(DEV), torch.from_numpy(tw).to(DEV))
    ref = O.moe_fake(x, ids, tw, gu, dn, dt)
    rv = ref.astype(np.float32) if dt == "fp16" else O.bf16_bits_to_f32(ref)
    err = _rel(_np(y.float()), rv)
    assert err <= 1e-3, err   # bar: rel. Frobenius error <= 1e-3


def test_moe_prequantized_input_equals_quantizing_first():
    """Routing pre-quantized rows (the runtime's pertoken_scale input) gives the bits of routing
    and quantizing the float rows in one step."""
    _say("moe prequant")
    x, ids, tw, q13, s13, q2, s2 = _moe_case(96, 256, 256, 4, seed=3)
    ops = _ops()
    qx, sx = ops.quant_per_token_i8(_t(x))
    a = ops.moe_permute_quant(_t(x), _t(ids), 4)
    b = ops.moe_permute_quant(qx, _t(ids), 4, x_scale=sx)
    for u, v in zip(a, b):
        assert torch.equal(u, v)
    y1 = ops.moe_w8a8_forward(_t(x), _t(ids), _t(tw), _t(q13), _t(s13), _t(q2), _t(s2))
    y2 = ops.moe_w8a8_forward(qx, _t(ids), _t(tw), _t(q13), _t(s13), _t(q2), _t(s2), out_dtype=torch.float16,
                              x_scale=sx)
    assert torch.equal(y1, y2)


def test_moe_mixtral_full_shape_sampled_tokens():
    """The Mixtral-shaped layer the bench measures (T = 512, H = 4096, I = 14336, E = 8, top-2;
    GEMM1 over 2I = 28672 > 10240 columns), runtime rule, checked on 34 sampled tokens against
    oracle.moe_runtime (per-token quantization makes every token independent): rel. Frobenius
    error <= 1e-3 and the routing offsets exact."""
    t, h, inter, e = 512, 4096, 14336, 8
    _say("moe mixtral full shape", t, h, inter, e)
    ops = _ops()
    gen = torch.Generator(device=DEV).manual_seed(11)
    rng = np.random.default_rng(12)
    x = torch.randn(t, h, generator=gen, device=DEV).half()
    ids, tw = O.mixtral_router(rng.standard_normal((t, e)).astype(np.float32), 2)
    q13, s13, _ = ops.w8_quantize_per_channel(
        (torch.randn(e * 2 * inter, h, generator=gen, device=DEV) * 0.02).half(), "export")
    q2, s2, _ = ops.w8_quantize_per_channel((torch.randn(e * h, inter, generator=gen, device=DEV) * 0.02).half(),
                                            "export")
    q13, s13 = q13.reshape(e, 2 * inter, h), s13.reshape(e, 2 * inter)
    q2, s2 = q2.reshape(e, h, inter), s2.reshape(e, h)
    y = ops.moe_w8a8_forward(x, _t(ids), _t(tw), q13, s13, q2, s2)
    torch.cuda.synchronize()
    _, _, _, offs = ops.moe_permute_quant(x, _t(ids), e)
    counts = np.bincount(ids.reshape(-1), minlength=e)
    assert np.array_equal(_np(offs), np.concatenate([[0], np.cumsum(counts)]))
    toks = np.unique(np.concatenate([rng.choice(t, 32, replace=False), [0, t - 1]]))
    ref = O.moe_runtime(_np(x)[toks], ids[toks], tw[toks], _np(q13), _np(s13), _np(q2), _np(s2))
    err = _rel(_np(y)[toks], ref)
    assert err <= 1e-3, err   # bar: rel. Frobenius error <= 1e-3


# Grouped GEMMs on crafted expert sizes (rows <= 256 per expert on average, the serving-size
# kernel): empty experts, one-row experts, experts of several 256-row chunks, more than 64
# experts, output widths that are not tile multiples.  (counts, k, n, inter)
GROUPED_CASES = [([0, 300, 1, 0, 130, 64], 256, 320, 96), ([128] * 4, 512, 256, 128), ([0, 0, 700], 128, 128, 64),
                 ([int(c) for c in np.random.default_rng(7).integers(0, 10, 70)], 256, 128, 64),
                 # longer K: experts of every size around the 32-row tile and 256-row chunk edges, weight
                 # slices past N and I, 70 experts, a K of 12 steps
                 ([0, 300, 1, 0, 130, 64, 257, 33, 31, 32, 256, 255], 512, 320, 96), ([128] * 4, 1024, 256, 128),
                 ([0, 0, 700], 512, 128, 64), ([int(c) for c in np.random.default_rng(8).integers(0, 10, 70)], 512, 128, 64),
                 ([31, 200, 17], 1536, 200, 200)]


@pytest.mark.parametrize("counts,k,n,inter", GROUPED_CASES)
def test_grouped_gemm_expert_sizes(counts, k, n, inter):
    _say("grouped", len(counts), sum(counts), k, n, inter)
    g = np.random.default_rng(sum(counts) + k)
    e, rows = len(counts), sum(counts)
    q = g.integers(-127, 128, (rows, k)).astype(np.int8)
    s = (g.random(rows) * 0.01 + 1e-3).astype(np.float32)
    w2 = g.integers(-127, 128, (e, n, k)).astype(np.int8)
    s2 = (g.random((e, n)) * 1e-3).astype(np.float32)
    w13 = g.integers(-127, 128, (e, 2 * inter, k)).astype(np.int8)
    s13 = (g.random((e, 2 * inter)) * 1e-3).astype(np.float32)
    offs = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    ops = _ops()
    y32 = _np(ops.moe_gmm2(_t(q), _t(s), _t(w2), _t(s2), _t(offs), torch.float32))
    y16 = _np(ops.moe_gmm2(_t(q), _t(s), _t(w2), _t(s2), _t(offs), torch.float16))
    qh, sh = ops.moe_gmm1_swiglu_quant(_t(q), _t(s), _t(w13), _t(s13), _t(offs), inter)
    qh, sh = _np(qh), _np(sh)
    agree = 0
    for ex in range(e):
        lo, hi = offs[ex], offs[ex + 1]
        if lo == hi:
            continue
        ref = O.w8a8_linear_runtime(q[lo:hi], s[lo:hi], w2[ex], s2[ex], out_dtype="fp32")
        assert np.array_equal(y32[lo:hi], ref), ex
        assert np.array_equal(y16[lo:hi], O.w8a8_linear_runtime(q[lo:hi], s[lo:hi], w2[ex], s2[ex])), ex
        acc = O.int_matmul_nt(q[lo:hi], w13[ex])
        gu = ((acc.astype(np.float32) * s[lo:hi][:, None]).astype(np.float32) * s13[ex][None, :]).astype(np.float32)
        hh = (O._silu(gu[:, :inter]) * gu[:, inter:]).astype(np.float32)
        rq, rs = O.quantize_per_token_runtime(hh, in_dtype="fp32")
        assert np.max(np.abs(qh[lo:hi].astype(int) - rq.astype(int))) <= 1, ex
        assert np.allclose(sh[lo:hi], rs, rtol=1e-6, atol=0), ex
        agree += np.sum(qh[lo:hi] == rq)
    assert agree / max(1, rows * inter) >= 0.999


# ------------------------------------------------------------------ fused add + RMSNorm + quant
# (m, h, residual): vector kernel (H % 8 == 0, 1 / 2 / 8 loads per thread, partial last load),
# three-pass kernel (H % 8 != 0)
NORM_CASES = [(1, 4096, True), (7, 4096, True), (64, 4096, False), (4, 12288, True), (2, 16384, True),
              (3, 5001, True), (5, 100, False)]


def _bits16(a):
    return np.ascontiguousarray(a).view(np.int16).astype(np.int32)


@pytest.mark.parametrize("m,h,res", NORM_CASES)
@pytest.mark.parametrize("dt", ["fp16", "bf16"])
def test_add_rms_norm_quant_matches_oracle(m, h, res, dt):
    _say("add_rms_norm_quant", m, h, res, dt)
    g = np.random.default_rng(h + m)
    xf = (g.standard_normal((m, h)) * 1.5).astype(np.float32)
    rf = g.standard_normal((m, h)).astype(np.float32)
    wf = (g.standard_normal(h) * 0.2 + 1).astype(np.float32)
    conv, tdt = ((lambda a: a.astype(np.float16)), torch.float16) if dt == "fp16" else (O.f32_to_bf16_bits,
                                                                                        torch.bfloat16)
    x, r, w = conv(xf), conv(rf), conv(wf)
    y_ref, _, _, r_ref = O.add_rms_norm_quant(x, r if res else None, w, 1e-6, dt)
    tx, tr, tw = _t(x, tdt), (_t(r, tdt) if res else None), _t(w, tdt)
    y, q, s, rs = _ops().add_rms_norm_quant(tx, tr, tw, 1e-6, quant=True, out=True)
    yb = _bits16(_np(y.view(torch.int16)))
    # residual sum: bit-exact (one fp32 add, one rounding)
    if res:
        assert np.array_equal(_bits16(_np(rs.view(torch.int16))), _bits16(r_ref))
    # y: only the fp32 summation order of the mean is free; one ulp of round(sum * rstd) can
    # become two after the weight multiply, so the bar is <= 2 units in the last place, and
    # almost every element is bit-identical
    d = np.abs(yb - _bits16(y_ref))
    assert d.max() <= 2 and np.mean(d == 0) >= 0.99
    # codes / scales: bit-exact to the per-token runtime quant of the kernel's own y, on the CPU
    # oracle and through the unfused GPU chain (mp_quant_per_token_i8)
    y_np = _np(y.view(torch.int16)).view(np.float16) if dt == "fp16" else _np(y.view(torch.int16)).view(np.uint16)
    q2, s2 = O.quantize_per_token_runtime(y_np, dt)
    assert np.array_equal(_np(q), q2) and np.array_equal(_np(s), s2)
    qq, ss = _ops().quant_per_token_i8(y)
    assert torch.equal(qq, q) and torch.equal(ss, s)
    # quant-only and in-place calls give the same bits
    y0, q0, s0, _ = _ops().add_rms_norm_quant(tx, tr, tw, 1e-6, quant=True, out=False)
    assert y0 is None and torch.equal(q0, q) and torch.equal(s0, s)
    xi, ri = tx.clone(), (tr.clone() if res else None)
    _ops().add_rms_norm_quant(xi, ri, tw, 1e-6, quant=False, inplace=True)
    assert torch.equal(xi, y)
    if res:
        assert torch.equal(ri, rs)
