"""The output-quant W8A8 linear (q/k/v ``quantize_output``, fake_quant.py:77-82, returned as
(int8, scale) like return_scale, vllm_ascend.patch:4019-4020): the GEMM epilogue writes y and each
row's partial abs-max, a second launch the codes.

Bars: y bit-exact against the oracle's runtime W8A8 linear; with the fp32 runtime rule the codes and
scales bit-exact against quantize_per_token_runtime of that (unfused) output; with the fake rule the
codes and scales bit-exact and fake values equal (up to the sign of zero) against
quantize_activation_per_token_fake of it.  Shapes cover
one token, decode batches, ragged M / N (row groups of 256, column slices of 128), bias / no bias, fp16
and bf16 outputs, and M = 4096 (16 row groups)."""
import sys

import numpy as np
import pytest
import torch

from oracle import quant as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _ops():
    from mindpipe_amd import ops
    return ops


def _u16(a):
    return np.asarray(a).view(np.uint16)


def _case(m, n, k, seed):
    rng = np.random.default_rng(seed)
    qx = rng.integers(-127, 128, (m, k), dtype=np.int8)
    qw = rng.integers(-127, 128, (n, k), dtype=np.int8)
    st = (rng.random(m) * 0.02 + 1e-4).astype(np.float32)
    sw = (rng.random(n) * 0.002 + 1e-5).astype(np.float32)
    if m > 2:
        qx[1] = 0  # an all-zero row: scale 0, codes 0 (runtime rule)
    return qx, qw, st, sw


CASES = [(1, 1280, 4096), (16, 12288, 4096), (7, 1000, 512), (300, 1000, 512), (257, 130, 128),
         (1000, 4096, 1024), (4096, 1536, 1024)]


@pytest.mark.parametrize("m,n,k", CASES)
@pytest.mark.parametrize("dt,odt", [(torch.float16, "fp16"), (torch.bfloat16, "bf16")])
@pytest.mark.parametrize("with_bias", [False, True])
def test_quant_out_runtime_rule_bit_exact(m, n, k, dt, odt, with_bias):
    _say("quant_out runtime", m, n, k, odt, with_bias)
    qx, qw, st, sw = _case(m, n, k, m + n + k)
    bias = (np.random.default_rng(9).standard_normal(n) * 0.1).astype(np.float16) if with_bias else None
    tb = None if bias is None else torch.from_numpy(bias).to(DEV)
    y, q, s = _ops().w8a8_gemm_quant_out(torch.from_numpy(qx).to(DEV), torch.from_numpy(st).to(DEV),
                                         torch.from_numpy(qw).to(DEV), torch.from_numpy(sw).to(DEV), tb, dt, False)
    yref = O.w8a8_linear_runtime(qx, st, qw, sw, bias, odt, "fp16")
    assert np.array_equal(_u16(y.view(torch.int16).cpu().numpy()), _u16(yref))
    qref, sref = O.quantize_per_token_runtime(yref, odt)
    assert np.array_equal(q.cpu().numpy(), qref)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), sref.view(np.uint32))


@pytest.mark.parametrize("m,n,k", [(16, 12288, 4096), (300, 1000, 512), (4096, 1536, 1024)])
@pytest.mark.parametrize("dt,odt", [(torch.float16, "fp16"), (torch.bfloat16, "bf16")])
def test_quant_out_fake_rule_bit_exact(m, n, k, dt, odt):
    _say("quant_out fake", m, n, k, odt)
    qx, qw, st, sw = _case(m, n, k, 3 * m + n)
    qx[1] = 1  # the fake rule's clamp path has its own test; keep rows non-zero here
    y, q, s = _ops().w8a8_gemm_quant_out(torch.from_numpy(qx).to(DEV), torch.from_numpy(st).to(DEV),
                                         torch.from_numpy(qw).to(DEV), torch.from_numpy(sw).to(DEV), None, dt, True)
    yref = O.w8a8_linear_runtime(qx, st, qw, sw, None, odt)
    assert np.array_equal(_u16(y.view(torch.int16).cpu().numpy()), _u16(yref))
    codes, sref, fake = O.quantize_activation_per_token_fake(yref, 8, odt)
    fake_k = (q.float() * s.unsqueeze(-1)).to(dt).float().cpu().numpy()
    # values, not bits: a zero code gives +0 where the reference's rint keeps the sign of -0.x
    fake_ref = fake.astype(np.float32) if odt == "fp16" else O.bf16_bits_to_f32(fake)
    # a bf16 row whose codes reach both +128 and -128 has no int8 form: the stored codes clamp one
    # side (the rule of quant_per_token_i8's bf16 fake path); only those elements may differ
    both = (codes.max(axis=1) == 128) & (codes.min(axis=1) == -128)
    diff = fake_k != fake_ref
    assert not diff[~both].any()
    assert np.all(np.abs(codes[diff]) == 128)
    if odt == "fp16":  # codes within +-127: stored as they are, with the fp16 scale
        assert np.array_equal(q.cpu().numpy().astype(np.int16), codes)
        assert np.array_equal(s.cpu().numpy(), sref.astype(np.float32))


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_smoothquant_linear_output_quant_fused_equals_unfused(dt):
    """SmoothQuantLinear(quantize_output=True): the fused path's fake output equals the unfused
    chain's (linear, then quantize_activation_per_token_absmax) bit for bit, and quantized_output
    returns that fake output's codes and scale."""
    _say("SmoothQuantLinear quantize_output", dt)
    from torch import nn
    from mindpipe_amd import ops
    from mindpipe_amd.smoothquant import SmoothQuantLinear, quantize_activation_per_token_absmax
    torch.manual_seed(0)
    lin = nn.Linear(512, 384, bias=True).to(dt).to(DEV)
    mod = SmoothQuantLinear.from_float(lin, quantize_output=True)
    x = torch.randn(2, 9, 512, device=DEV).to(dt)
    out = mod(x)
    fake, q, s = mod._input_codes(x)
    y = mod._linear(x, fake, q, s)
    ref = quantize_activation_per_token_absmax(y)
    assert torch.equal(out, ref)
    qo, so = mod.quantized_output(x)
    assert qo.shape == (2, 9, 384) and so.shape == (2, 9)
    assert torch.equal((qo.float() * so.unsqueeze(-1)).to(dt), out)
