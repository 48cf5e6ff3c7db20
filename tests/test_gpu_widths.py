"""GPU tests of the quantizers and modules at code widths other than W8A8 / W4, against the
reference's own outputs (``golden/reference_width_vectors.npz``, written by
``golden/make_width_vectors.py`` from the reference functions and modules).

* AWQ ``pseudo_quantize_tensor`` at 2, 3 and 8 bits and the fake per-token / per-channel
  quantizers at 3, 4 and 6 bits: bit-exact (every op rounds as the reference's).
* ``SmoothQuantLinear`` at W4A8, W8A4, W6A6, W8A16, W16A8, W16A16 and W4A4: relative Frobenius
  error <= 1e-3 without output quant.  With output quant (W6A6, W4A4) the output codes are
  coarse: a one-ulp difference of the pre-quant output (fp32 summation order) can move a value
  to the next code, so the bar there is: at most 2% of the values differ, each by at most one
  output quantization step of its row.
* ``SmoothQuantPackedMoeExperts`` at W4A4 / SiLU, W8A8 / tanh-GELU, W8A16 / SiLU and
  W6A6 / tanh-GELU (the expert loop): the intermediate per-token requant is coarse as above,
  so the bar is a relative Frobenius error <= 2e-2 and, for W8A16 (no requant), <= 1e-3.
"""
from pathlib import Path

import numpy as np
import pytest
import torch
from torch import nn

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
WID = np.load(Path(__file__).parent / "golden" / "reference_width_vectors.npz")
DTS = [(torch.float16, "f16"), (torch.bfloat16, "bf16")]


def _say(*a):
    print(*a, flush=True)


def _t(key, dt):
    a = WID[key]
    t = torch.from_numpy(np.ascontiguousarray(a))
    return (t.view(torch.bfloat16) if dt == torch.bfloat16 else t).to(DEV)


def _bits(t):
    return t.detach().contiguous().view(torch.int16).cpu()


def _rel(y, ref):
    return ((y.float() - ref.float()).norm() / ref.float().norm()).item()


@pytest.mark.parametrize("dt,tag", DTS)
def test_awq_other_widths_bit_exact(dt, tag):
    from mindpipe_amd.w4a16 import pseudo_quantize_tensor
    w = _t(f"awq_{tag}_w", dt)
    n = 0
    for n_bit in (2, 3, 8):
        for zp in (True, False):
            for g in (128, -1):
                key = f"awq_{tag}_n{n_bit}_zp{int(zp)}_g{g}"
                if key + "_deq" not in WID.files:
                    continue
                _say("awq", key)
                if zp:
                    d, s, z = pseudo_quantize_tensor(w.clone(), n_bit=n_bit, zero_point=True, q_group_size=g,
                                                     get_scale_zp=True)
                    assert torch.equal(_bits(s), _bits(_t(key + "_s", dt))), key
                    assert torch.equal(_bits(z), _bits(_t(key + "_z", dt))), key
                else:
                    d = pseudo_quantize_tensor(w.clone(), n_bit=n_bit, zero_point=False, q_group_size=g)
                assert torch.equal(_bits(d), _bits(_t(key + "_deq", dt))), key
                n += 1
    assert n == 8


@pytest.mark.parametrize("dt,tag", DTS)
def test_fake_quantizers_other_widths_bit_exact(dt, tag):
    from mindpipe_amd.smoothquant import quantize_activation_per_token_absmax, quantize_weight_per_channel_absmax
    x, w = _t(f"fq_{tag}_x", dt), _t(f"fq_{tag}_w", dt)
    # values, not bits: a code of 0 times a scale is +0 here and -0 in the reference where the
    # input was negative (int8 codes carry no sign of zero)
    for n in (3, 4, 6):
        _say("fake quant", tag, n)
        assert torch.equal(quantize_activation_per_token_absmax(x, n).float(), _t(f"fq_{tag}_x_n{n}", dt).float())
        assert torch.equal(quantize_weight_per_channel_absmax(w, n).float(), _t(f"fq_{tag}_w_n{n}", dt).float())


LIN_CFGS = [(4, 8, False), (8, 4, False), (6, 6, True), (8, 16, False), (16, 8, False), (16, 16, False),
            (4, 4, True)]


@pytest.mark.parametrize("dt,tag", DTS)
@pytest.mark.parametrize("wb,ab,qo", LIN_CFGS)
def test_smoothquant_linear_other_widths(dt, tag, wb, ab, qo):
    from mindpipe_amd.smoothquant import SmoothQuantLinear
    _say("linear", tag, wb, ab, qo)
    lin = nn.Linear(256, 96, bias=True).to(device=DEV, dtype=dt)
    with torch.no_grad():
        lin.weight.copy_(_t(f"lin_{tag}_w", dt))
        lin.bias.copy_(_t(f"lin_{tag}_b", dt))
    x = _t(f"lin_{tag}_x", dt)
    mod = SmoothQuantLinear.from_float(lin, wb, ab, quantize_output=qo)
    assert repr(mod).startswith(f"SmoothQuantLinear(256, 96, bias=True, weight_bits={wb}, activation_bits={ab}")
    y = mod(x)
    ref = _t(f"lin_{tag}_w{wb}a{ab}q{int(qo)}_y", dt)
    assert y.shape == ref.shape and y.dtype == ref.dtype
    if not qo:
        assert _rel(y, ref) <= 1e-3
        return
    # output quant at ab bits: compare value by value against the row's quantization step
    q_max = 2 ** (ab - 1) - 1
    step = ref.float().abs().amax(dim=-1, keepdim=True) / q_max
    diff = (y.float() - ref.float()).abs()
    assert (diff <= step * 1.01 + 1e-6).all()
    assert (diff > 0).float().mean().item() <= 0.02
    # the codes path of the same module agrees with its forward
    q, s = mod.quantized_output(x)
    assert torch.equal((q.float() * s.unsqueeze(-1)).to(dt).float(), y.reshape(-1, 96).float())


MOE_CFGS = [(4, 4, "silu"), (8, 8, "gelu_tanh"), (8, 16, "silu"), (6, 6, "gelu_tanh")]


@pytest.mark.parametrize("dt,tag", DTS)
@pytest.mark.parametrize("wb,ab,act", MOE_CFGS)
def test_packed_moe_other_widths_and_activations(dt, tag, wb, ab, act):
    from mindpipe_amd.smoothquant import SmoothQuantPackedMoeExperts
    _say("moe", tag, wb, ab, act)
    acts = {"silu": nn.SiLU(), "gelu_tanh": nn.GELU(approximate="tanh")}
    gu, dn, x = _t(f"moe_{tag}_gu", dt), _t(f"moe_{tag}_dn", dt), _t(f"moe_{tag}_x", dt)
    ids = torch.from_numpy(WID[f"moe_{tag}_ids"]).long().to(DEV)
    tw = _t(f"moe_{tag}_tw", dt)
    mod = SmoothQuantPackedMoeExperts(gu, dn, acts[act], weight_bits=wb, activation_bits=ab)
    y = mod(x, ids, tw)
    ref = _t(f"moe_{tag}_w{wb}a{ab}_{act}_y", dt)
    assert y.shape == ref.shape and y.dtype == ref.dtype
    assert _rel(y, ref) <= (1e-3 if ab >= 16 else 2e-2)


def test_widths_outside_int8_codes_raise():
    from mindpipe_amd.smoothquant import SmoothQuantLinear, quantize_activation_per_token_absmax
    from mindpipe_amd.w4a16 import pseudo_quantize_tensor
    x = torch.randn(4, 64, device=DEV).half()
    with pytest.raises(NotImplementedError):
        quantize_activation_per_token_absmax(x, 12)
    with pytest.raises(NotImplementedError):
        SmoothQuantLinear(64, 32, weight_bits=10)
    with pytest.raises(NotImplementedError):
        pseudo_quantize_tensor(x.clone(), n_bit=9)
    with pytest.raises(ValueError):
        SmoothQuantLinear(64, 32, weight_bits=4, scale_rule="export")
