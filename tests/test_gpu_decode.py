"""GPU tests of the decode-step harness kernels (RoPE + KV append, split-K decode
attention with its in-launch split merge, the fused RoPE + append + attention
launch, SiLU-mul) and of one decoder step on them against the PyTorch step.

Bars: RoPE and the cache writes are bit-exact to the same fp16 op sequence in
PyTorch; attention has relative Frobenius error <= 1e-3 against fp32 softmax
attention; SiLU-mul is within one fp16 ulp (exp is not correctly rounded on
either side); decoder logits within 2e-2 relative of the PyTorch step (the
RMSNorm statistics differ by design: fp32 sum vs the rounded residual).  The PyTorch
step shares no kernel with the HIP step: its linears are F.linear on the
pseudo-quantized fp16 weights unpacked with torch bit operations, its norms, RoPE and
attention are torch ops."""
import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _say(*a):
    print(*a, flush=True)


def _rel(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _tables(cap, hd=128, theta=10000.0):
    inv = 1.0 / (theta ** (torch.arange(0, hd, 2, device=DEV).float() / hd))
    f = torch.outer(torch.arange(cap, device=DEV).float(), inv)
    return f.cos().half(), f.sin().half()


def _rope_torch(x, cos, sin):
    x1, x2 = x[..., 0::2], x[..., 1::2]
    out = torch.empty_like(x)
    out[..., 0::2] = x1 * cos - x2 * sin
    out[..., 1::2] = x1 * sin + x2 * cos
    return out


@pytest.mark.parametrize("b,nh,kvh,pos", [(1, 4, 4, 0), (3, 8, 2, 37), (2, 8, 1, 63)])
def test_rope_append_bit_exact(b, nh, kvh, pos):
    _say("rope_append", b, nh, kvh, pos)
    from mindpipe_amd import ops
    cap, hd = 64, 128
    g = torch.Generator(device=DEV).manual_seed(1)
    qkv = torch.randn(b, (nh + 2 * kvh) * hd, device=DEV, generator=g).half()
    cos, sin = _tables(cap)
    kc = torch.zeros(b, kvh, cap, hd, device=DEV, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    p = torch.tensor([pos], device=DEV, dtype=torch.int64)
    q = ops.decode_rope_append(qkv, nh, kvh, cos, sin, p, kc, vc)
    heads = qkv.reshape(b, nh + 2 * kvh, hd)
    assert torch.equal(q, _rope_torch(heads[:, :nh], cos[pos], sin[pos]))
    assert torch.equal(kc[:, :, pos], _rope_torch(heads[:, nh:nh + kvh], cos[pos], sin[pos]))
    assert torch.equal(vc[:, :, pos], heads[:, nh + kvh:])
    others = torch.ones(cap, dtype=torch.bool, device=DEV)
    others[pos] = False
    assert not kc[:, :, others].any() and not vc[:, :, others].any()
    # a position outside the cache writes nothing
    k0, v0 = kc.clone(), vc.clone()
    ops.decode_rope_append(qkv, nh, kvh, cos, sin, torch.tensor([cap], device=DEV), kc, vc)
    assert torch.equal(kc, k0) and torch.equal(vc, v0)


@pytest.mark.parametrize("b,t,nh,kvh,cap", [(1, 5, 4, 4, 8), (2, 37, 8, 2, 64), (3, 64, 8, 1, 64), (1, 300, 32, 32, 301)])
def test_prefill_rope_split_bit_exact(b, t, nh, kvh, cap):
    """The prefill split of the fused qkv rows: rotated queries in [B, nh, T, 128], rotated keys and the
    values in cache rows 0 .. T-1 (rows past T untouched), against the torch fp16 RoPE."""
    _say("prefill_rope_split", b, t, nh, kvh, cap)
    from mindpipe_amd import ops
    hd = 128
    g = torch.Generator(device=DEV).manual_seed(3)
    qkv = torch.randn(b * t, (nh + 2 * kvh) * hd, device=DEV, generator=g).half()
    cos, sin = _tables(cap)
    kc = torch.full((b, kvh, cap, hd), 7.0, device=DEV, dtype=torch.float16)
    vc = torch.full_like(kc, -7.0)
    q = ops.prefill_rope_split(qkv, b, nh, kvh, cos, sin, kc, vc)
    heads = qkv.reshape(b, t, nh + 2 * kvh, hd).transpose(1, 2)  # [B, heads, T, hd]
    c, s_ = cos[:t].unsqueeze(0).unsqueeze(0), sin[:t].unsqueeze(0).unsqueeze(0)
    assert torch.equal(q, _rope_torch(heads[:, :nh], c, s_))
    assert torch.equal(kc[:, :, :t], _rope_torch(heads[:, nh:nh + kvh], c, s_))
    assert torch.equal(vc[:, :, :t], heads[:, nh + kvh:])
    assert bool((kc[:, :, t:] == 7.0).all()) and bool((vc[:, :, t:] == -7.0).all())


@pytest.mark.parametrize("b,nh,kvh,cap,pos,splits", [(1, 4, 4, 300, 0, 8), (2, 8, 2, 300, 299, 1),
                                                     (3, 8, 1, 257, 130, 5), (1, 16, 2, 2304, 2200, 32),
                                                     (2, 4, 4, 1000, 511, 3)])
def test_decode_attention_matches_fp32(b, nh, kvh, cap, pos, splits):
    _say("decode_attention", b, nh, kvh, cap, pos, splits)
    from mindpipe_amd import ops
    hd = 128
    g = torch.Generator(device=DEV).manual_seed(2)
    q = torch.randn(b, nh, hd, device=DEV, generator=g).half()
    kc = torch.randn(b, kvh, cap, hd, device=DEV, generator=g).half()
    vc = torch.randn(b, kvh, cap, hd, device=DEV, generator=g).half()
    scale = 1.0 / math.sqrt(hd)
    ws = ops.decode_attention_workspace(b, nh, splits, DEV)
    out = ops.decode_attention(q, kc, vc, torch.tensor([pos], device=DEV), splits, scale, ws)
    grp = nh // kvh
    qf = q.float().reshape(b, kvh, grp, hd)
    kf = kc[:, :, :pos + 1].float()
    s = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * scale
    ref = torch.matmul(torch.softmax(s, -1), vc[:, :, :pos + 1].float()).reshape(b, nh, hd)
    err = _rel(out.float(), ref)
    assert err <= 1e-3, err


@pytest.mark.parametrize("b,nh,kvh,cap,pos,splits", [(1, 4, 4, 300, 0, 8), (2, 8, 2, 300, 299, 1),
                                                     (3, 8, 1, 257, 130, 5), (1, 32, 32, 2304, 2047, 32),
                                                     (1, 64, 8, 4096, 4000, 100), (2, 16, 2, 640, 64, 10),
                                                     # head groups on MFMA: two 64-position steps, the
                                                     # appended row in the second
                                                     (1, 32, 4, 1024, 1000, 8), (2, 32, 8, 512, 383, 4)])
def test_decode_rope_attention_equals_two_launch_path(b, nh, kvh, cap, pos, splits):
    """The fused RoPE + append + attention launch writes the same cache rows and the
    same output bits as rope_append followed by attention (one kernel body)."""
    _say("decode_rope_attention", b, nh, kvh, cap, pos, splits)
    from mindpipe_amd import ops
    hd = 128
    g = torch.Generator(device=DEV).manual_seed(4)
    qkv = torch.randn(b, (nh + 2 * kvh) * hd, device=DEV, generator=g).half()
    cos, sin = _tables(cap)
    kc = torch.randn(b, kvh, cap, hd, device=DEV, generator=g).half()
    vc = torch.randn(b, kvh, cap, hd, device=DEV, generator=g).half()
    k2, v2 = kc.clone(), vc.clone()
    p = torch.tensor([pos], device=DEV, dtype=torch.int64)
    scale = 1.0 / math.sqrt(hd)
    ws = ops.decode_attention_workspace(b, nh, splits, DEV)
    out = ops.decode_rope_attention(qkv, nh, kvh, cos, sin, p, kc, vc, splits, scale, ws)
    q = ops.decode_rope_append(qkv, nh, kvh, cos, sin, p, k2, v2)
    ref = ops.decode_attention(q, k2, v2, p, splits, scale, ws)
    assert torch.equal(kc, k2) and torch.equal(vc, v2)
    assert torch.equal(out, ref)
    # a second call gives the same bits
    out2 = ops.decode_rope_attention(qkv, nh, kvh, cos, sin, p, kc, vc, splits, scale, ws)
    assert torch.equal(out2, out)
    # and the fp32 attention over [0, pos] agrees
    grp = nh // kvh
    qf = q.float().reshape(b, kvh, grp, hd)
    s = torch.matmul(qf, kc[:, :, :pos + 1].float().transpose(-1, -2).contiguous()) * scale
    want = torch.matmul(torch.softmax(s, -1), vc[:, :, :pos + 1].float()).reshape(b, nh, hd)
    assert _rel(out.float(), want) <= 1e-3


def test_decode_attention_workspace_reuse_and_edges():
    """One workspace across calls with different used-split counts; an empty range
    gives zeros; a position outside the cache appends nothing and gives zeros in the
    fused launch."""
    _say("decode_attention workspace reuse")
    from mindpipe_amd import ops
    b, nh, kvh, cap, hd, splits = 2, 8, 2, 500, 128, 16
    g = torch.Generator(device=DEV).manual_seed(5)
    kc = torch.randn(b, kvh, cap, hd, device=DEV, generator=g).half()
    vc = torch.randn(b, kvh, cap, hd, device=DEV, generator=g).half()
    q = torch.randn(b, nh, hd, device=DEV, generator=g).half()
    scale = 1.0 / math.sqrt(hd)
    ws = ops.decode_attention_workspace(b, nh, splits, DEV)
    grp = nh // kvh
    for pos in [499, 3, 40, 0, 250, 31, 32, 499]:
        out = ops.decode_attention(q, kc, vc, torch.tensor([pos], device=DEV), splits, scale, ws)
        qf = q.float().reshape(b, kvh, grp, hd)
        s = torch.matmul(qf, kc[:, :, :pos + 1].float().transpose(-1, -2).contiguous()) * scale
        want = torch.matmul(torch.softmax(s, -1), vc[:, :, :pos + 1].float()).reshape(b, nh, hd)
        assert _rel(out.float(), want) <= 1e-3, pos
    out = ops.decode_attention(q, kc, vc, torch.tensor([-1], device=DEV), splits, scale, ws)
    assert not out.any()
    qkv = torch.randn(b, (nh + 2 * kvh) * hd, device=DEV, generator=g).half()
    cos, sin = _tables(cap)
    k0, v0 = kc.clone(), vc.clone()
    out = ops.decode_rope_attention(qkv, nh, kvh, cos, sin, torch.tensor([cap], device=DEV), kc, vc, splits,
                                    scale, ws)
    assert not out.any() and torch.equal(kc, k0) and torch.equal(vc, v0)


def test_silu_mul_within_one_ulp():
    _say("silu_mul")
    from mindpipe_amd import ops
    gu = (torch.randn(5, 2 * 1000, device=DEV, generator=torch.Generator(device=DEV).manual_seed(3)) * 3).half()
    act = ops.silu_mul(gu)
    ref = torch.nn.functional.silu(gu[:, :1000]) * gu[:, 1000:]
    d = (act.view(torch.int16).int() - ref.view(torch.int16).int()).abs()
    assert int(d.max()) <= 1 and float((d == 0).float().mean()) >= 0.99


def test_silu_mul_bf16_within_one_ulp():
    """bf16 silu_mul against torch's bf16 ops (silu in fp32 rounded to bf16, the product rounded)."""
    _say("silu_mul bf16")
    from mindpipe_amd import ops
    gu = (torch.randn(5, 2 * 1000, device=DEV, generator=torch.Generator(device=DEV).manual_seed(4)) * 3).bfloat16()
    act = ops.silu_mul(gu)
    assert act.dtype == torch.bfloat16
    ref = torch.nn.functional.silu(gu[:, :1000]) * gu[:, 1000:]
    d = (act.view(torch.int16).int() - ref.view(torch.int16).int()).abs()
    assert int(d.max()) <= 1 and float((d == 0).float().mean()) >= 0.99


@pytest.mark.parametrize("heads,kv_heads", [(2, 2), (4, 1)])
def test_decoder_prefill_matches_torch_prefill(heads, kv_heads):
    _say("decoder prefill", heads, kv_heads)
    from mindpipe_amd.decoder import DecoderConfig, W4Decoder
    cfg = DecoderConfig(layers=2, hidden=heads * 128, heads=heads, kv_heads=kv_heads, ffn=512, vocab=512)
    model = W4Decoder(cfg, max_batch=2, max_len=96, device=DEV, seed=5)
    toks = torch.randint(0, cfg.vocab, (2, 70), device=DEV, generator=torch.Generator(device=DEV).manual_seed(6))
    lk = model.prefill(toks, return_logits=True)
    kc, vc = model.k_cache.clone(), model.v_cache.clone()
    lt = model.prefill_torch(toks, return_logits=True)
    # fused kernels vs PyTorch ops (fp32 attention in the reference): same math, other roundings
    assert _rel(lk.float(), lt.float()) <= 2e-2
    assert _rel(kc.float(), model.k_cache.float()) <= 1e-2 and _rel(vc.float(), model.v_cache.float()) <= 1e-2


@pytest.mark.parametrize("heads,kv_heads", [(2, 2), (4, 1)])
def test_decoder_kernel_step_matches_torch_step(heads, kv_heads):
    _say("decoder step", heads, kv_heads)
    from mindpipe_amd.decoder import DecoderConfig, W4Decoder
    cfg = DecoderConfig(layers=2, hidden=heads * 128, heads=heads, kv_heads=kv_heads, ffn=512, vocab=512)
    model = W4Decoder(cfg, max_batch=2, max_len=96, device=DEV, seed=3)
    g = torch.Generator(device=DEV).manual_seed(4)
    toks = torch.randint(0, cfg.vocab, (2, 40), device=DEV, generator=g)
    model.prefill(toks)
    tok = torch.randint(0, cfg.vocab, (2,), device=DEV, generator=g)
    cur = torch.tensor([40], device=DEV, dtype=torch.int64)
    lk = model.decode_step(tok, cur, return_logits=True)
    lt = model.decode_step_torch(tok, cur, return_logits=True)
    err = _rel(lk.float(), lt.float())
    assert err <= 2e-2, err


@pytest.mark.parametrize("k,n,swiglu,res,bias,zp", [(4096, 12288, False, True, False, True),
                                                    (4096, 2 * 1000, True, True, False, True),
                                                    (2048, 300, False, False, True, False),
                                                    (8192, 1100, False, True, True, True),
                                                    (8192, 2 * 700, True, False, False, True),
                                                    (2048, 2 * 64, True, True, True, False)])
def test_gemv_add_rms_norm_equals_two_launch_chain(k, n, swiglu, res, bias, zp):
    """The norm-fused one-row GEMV against add_rms_norm_quant (quant off) followed by w4a16_gemm /
    w4a16_gemm_swiglu: the same residual sum bits, and the same output bits where the second step runs
    the same VALU GEMV arithmetic (the fused gate/up, K = 8192); where w4a16_gemm takes the
    matrix-core GEMV (one row, K = 2048 / 4096: another summation order) rel. error <= 1e-3."""
    _say("gemv_add_rms_norm", k, n, swiglu, res, bias, zp)
    from mindpipe_amd import ops
    g = torch.Generator(device=DEV).manual_seed(k + n)
    x = torch.randn(1, k, device=DEV, generator=g).half()
    r = torch.randn(1, k, device=DEV, generator=g).half() if res else None
    w = (1.0 + 0.1 * torch.randn(k, device=DEV, generator=g)).half()
    packed = torch.randint(-2**31, 2**31 - 1, (n, k // 8), device=DEV, dtype=torch.int32, generator=g)
    sc = (torch.rand(n, k // 128, device=DEV, generator=g) * 0.002 + 0.001).half()
    zr = torch.randint(0, 16, (n, k // 128), device=DEV, generator=g).half() if zp else None
    b = torch.randn(n, device=DEV, generator=g).half() if bias else None
    y, rsum = ops.w4a16_gemv_add_rms_norm(x, r, w, 1e-5, packed, sc, zr, 128, b, swiglu)
    hn, _, _, rs2 = ops.add_rms_norm_quant(x, r, w, 1e-5, quant=False)
    want = (ops.w4a16_gemm_swiglu(hn, packed, sc, zr, 128, b) if swiglu
            else ops.w4a16_gemm(hn, packed, sc, zr, 128, b))
    if swiglu or k not in (2048, 4096):
        assert torch.equal(y, want)
    else:
        assert _rel(y.float(), want.float()) <= 1e-3
    assert (rsum is None) == (r is None) and (rsum is None or torch.equal(rsum, rs2))
    # a second call (other workgroup timing) gives the same bits
    y2, _ = ops.w4a16_gemv_add_rms_norm(x, r, w, 1e-5, packed, sc, zr, 128, b, swiglu)
    assert torch.equal(y2, y)


def test_gemv_add_rms_norm_rejects_unsupported():
    from mindpipe_amd import ops
    x = torch.randn(1, 1024, device=DEV).half()
    w = torch.ones(1024, device=DEV).half()
    packed = torch.zeros(64, 128, device=DEV, dtype=torch.int32)
    sc = torch.ones(64, 8, device=DEV).half()
    with pytest.raises(RuntimeError):
        ops.w4a16_gemv_add_rms_norm(x, None, w, 1e-5, packed, sc, None, 128)  # K = 1024
    with pytest.raises(RuntimeError):  # more than one row
        ops.w4a16_gemv_add_rms_norm(torch.randn(2, 2048, device=DEV).half(), None, torch.ones(2048, device=DEV).half(),
                                    1e-5, torch.zeros(64, 256, device=DEV, dtype=torch.int32),
                                    torch.ones(64, 16, device=DEV).half(), None, 128)


def test_decoder_one_row_step_fused_norm():
    """B = 1 decode step with every add-RMSNorm inside the next GEMV: within 1e-3 of the two-launch
    chain (whose q/k/v GEMV at K = 2048 runs the matrix-core GEMV, another summation order than the
    norm-fused VALU GEMV), and within 2e-2 of the PyTorch step."""
    _say("decoder fused-norm step")
    from mindpipe_amd.decoder import DecoderConfig, W4Decoder
    cfg = DecoderConfig(layers=2, hidden=2048, heads=16, kv_heads=4, ffn=1024, vocab=512)
    model = W4Decoder(cfg, max_batch=1, max_len=96, device=DEV, seed=7)
    g = torch.Generator(device=DEV).manual_seed(8)
    toks = torch.randint(0, cfg.vocab, (1, 40), device=DEV, generator=g)
    model.prefill(toks)
    kc, vc = model.k_cache.clone(), model.v_cache.clone()
    tok = torch.randint(0, cfg.vocab, (1,), device=DEV, generator=g)
    cur = torch.tensor([40], device=DEV, dtype=torch.int64)
    lf = model.decode_step(tok, cur, return_logits=True)
    model.k_cache.copy_(kc); model.v_cache.copy_(vc)
    model.fuse_norm = False
    lu = model.decode_step(tok, cur, return_logits=True)
    assert _rel(lf.float(), lu.float()) <= 1e-3
    model.k_cache.copy_(kc); model.v_cache.copy_(vc)
    lt = model.decode_step_torch(tok, cur, return_logits=True)
    assert _rel(lf.float(), lt.float()) <= 2e-2


@pytest.mark.parametrize("rows,n", [(1, 32000), (8, 128256), (3, 1), (5, 1500), (4, 20001), (2, 16384),
                                    (6, 16383)])
def test_argmax_rows_matches_torch(rows, n):
    """Row argmax equals torch.argmax, including ties (first index; across the 4096-value spans of
    the split form), all -inf rows, NaN, and +0 / -0 ties.  Rows of 16384+ values take the split
    form (16-byte loads when n % 8 == 0, scalar loads otherwise); shorter rows one workgroup each."""
    _say("argmax_rows", rows, n)
    from mindpipe_amd import ops
    g = torch.Generator(device=DEV).manual_seed(rows * 7 + n)
    x = torch.randn(rows, n, device=DEV, generator=g).half()
    if n > 100:
        x[0, 17] = 30.0
        x[0, n - 5] = 30.0                      # tie: the lower index wins
    if rows > 2:
        x[1] = float("-inf")                     # all equal: index 0
        x[2, n // 2] = float("nan")              # NaN counts as the maximum
    if rows > 3:
        x[2, n - 1] = float("nan")               # a later NaN loses to the first
        x[3] = 0.0
        x[3, : n // 2] = -0.0                    # -0 and +0 are equal: index 0
    assert torch.equal(ops.argmax_rows(x), torch.argmax(x, dim=-1))


def test_decode_ops_reject_wrong_extents():
    """The decode ops check every extent the kernels assume before launching (the C ABI sees only
    pointers): qkv width, cache shapes, RoPE table rows, pos, output and workspace."""
    _say("decode op checks")
    from mindpipe_amd import ops
    b, nh, kvh, cap = 2, 4, 2, 64
    qkv = torch.zeros(b, (nh + 2 * kvh) * 128, device=DEV).half()
    kc = torch.zeros(b, kvh, cap, 128, device=DEV).half()
    vc = torch.zeros_like(kc)
    cos = torch.zeros(cap, 64, device=DEV).half()
    sin = torch.zeros_like(cos)
    pos = torch.tensor([3], device=DEV, dtype=torch.int64)
    ws = ops.decode_attention_workspace(b, nh, 1, DEV)
    ops.decode_rope_attention(qkv, nh, kvh, cos, sin, pos, kc, vc, 1, 0.1, ws)   # the valid call
    bad = [
        lambda: ops.decode_rope_attention(qkv[:, :-128].contiguous(), nh, kvh, cos, sin, pos, kc, vc, 1, 0.1, ws),
        lambda: ops.decode_rope_attention(qkv, nh, kvh, cos[:cap - 1].contiguous(), sin, pos, kc, vc, 1, 0.1, ws),
        lambda: ops.decode_rope_attention(qkv, nh, kvh, cos, sin, pos, kc[:1].contiguous(), vc, 1, 0.1, ws),
        lambda: ops.decode_rope_attention(qkv, nh, kvh, cos, sin, pos.int(), kc, vc, 1, 0.1, ws),
        lambda: ops.decode_rope_attention(qkv, nh, kvh, cos, sin, torch.tensor([1, 2], device=DEV), kc, vc, 1, 0.1, ws),
        lambda: ops.decode_rope_append(qkv, nh, 3, cos, sin, pos, kc, vc),
        lambda: ops.decode_attention(torch.zeros(b, nh, 64, device=DEV).half(), kc, vc, pos, 1, 0.1, ws),
        lambda: ops.decode_attention(torch.zeros(b, nh, 128, device=DEV).half(), kc, vc[..., :64].contiguous(), pos,
                                     1, 0.1, ws),
        lambda: ops.decode_rope_attention(qkv, nh, kvh, cos, sin, pos, kc, vc, 1, 0.1, ws,
                                          out=torch.empty(b, nh + 1, 128, device=DEV).half()),
    ]
    for i, f in enumerate(bad):
        with pytest.raises(RuntimeError):
            f()
        torch.cuda.synchronize()
