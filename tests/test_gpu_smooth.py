"""GPU parity of the SmoothQuant smoothing kernels and their Python API.

* ``compute_smooth_scales`` against the reference's own ``_compute_smooth_scales`` outputs
  (``tests/golden`` vectors, fp16 and bf16, alpha 0.5): bit-exact; and against the oracle at
  K = 4096 for alpha 0.5 and 0.85: bit-exact.
* ``colmax_abs`` (the statistic of both ``get_act_scales`` and the weight side) against numpy:
  exact, with accumulation across calls, ragged K and fp32 input.
* ``smooth_ln_fcs_llama_like``: norm and fc weights equal to the closed forms R(ln / s), R(w * s).
* ``get_act_scales`` on a tiny HF Llama: equal to the max over the same hooks computed with torch;
  ``smooth_lm`` leaves the model function unchanged to fp16 rounding (the smoothing identity).
"""
import sys
from pathlib import Path

import numpy as np
import pytest
import torch
from torch import nn

from oracle import quant as O

pytestmark = pytest.mark.gpu
EXT = np.load(Path(__file__).parent / "golden" / "reference_ext_vectors.npz")
DEV = "cuda:0"


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _lin_from(w: np.ndarray, dt):
    n, k = w.shape
    fc = nn.Linear(k, n, bias=False).to(dt).to(DEV)
    with torch.no_grad():
        fc.weight.copy_(torch.from_numpy(w).view(dt).to(DEV))
    return fc


@pytest.mark.parametrize("tag,dt,odt", [("f16", torch.float16, "fp16"), ("bf16", torch.bfloat16, "bf16")])
def test_smooth_scales_match_reference_vectors(tag, dt, odt):
    _say("smooth scales ref", tag)
    from mindpipe_amd.smoothquant import compute_smooth_scales
    w0, w1 = EXT[f"smooth_{tag}_w0"], EXT[f"smooth_{tag}_w1"]
    if odt == "bf16":
        w0, w1 = w0.view(np.int16), w1.view(np.int16)
    fcs = [_lin_from(w0, dt), _lin_from(w1, dt)]
    s = compute_smooth_scales(fcs, torch.from_numpy(EXT[f"smooth_{tag}_a"]), 0.5)
    assert s.dtype == dt
    got = s.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, EXT[f"smooth_{tag}_s"].view(np.uint16))


@pytest.mark.parametrize("alpha", [0.5, 0.85])
@pytest.mark.parametrize("dt,odt", [(torch.float16, "fp16"), (torch.bfloat16, "bf16")])
def test_smooth_scales_match_oracle_at_4096(alpha, dt, odt):
    _say("smooth scales oracle", alpha, odt)
    from mindpipe_amd.smoothquant import compute_smooth_scales
    rng = np.random.default_rng(3)
    k = 4096
    a = np.abs(rng.standard_normal(k)).astype(np.float32) * 4
    a[rng.choice(k, 40, replace=False)] *= 50            # outlier channels
    a[:3] = 0.0                                         # clamp of the result
    ws = [(rng.standard_normal((n, k)) * 0.02).astype(np.float32) for n in (1024, 512, 256)]
    ws[0][:, 5] = 0.0                                   # clamped weight column
    if odt == "fp16":
        wn = [w.astype(np.float16) for w in ws]
        fcs = [_lin_from(w, dt) for w in wn]
    else:
        wn = [O.f32_to_bf16_bits(w) for w in ws]
        fcs = [_lin_from(w.view(np.int16), dt) for w in wn]
    ref = O.compute_smooth_scales(a, wn, alpha, odt)
    s = compute_smooth_scales(fcs, torch.from_numpy(a), alpha)
    got = s.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, np.asarray(ref).view(np.uint16))


@pytest.mark.parametrize("rows,k,dt", [(1000, 4096, torch.float16), (37, 1000, torch.bfloat16), (5, 13, torch.float32),
                                       (3000, 520, torch.float16)])
def test_colmax_abs_exact_and_accumulates(rows, k, dt):
    _say("colmax", rows, k, dt)
    from mindpipe_amd import ops
    g = torch.Generator(device=DEV).manual_seed(rows + k)
    x1 = torch.randn(rows, k, device=DEV, generator=g).to(dt)
    x2 = (torch.randn(rows // 2 + 1, k, device=DEV, generator=g) * 3).to(dt)
    cm = ops.colmax_abs(x1)
    want1 = x1.float().abs().amax(dim=0)
    assert torch.equal(cm, want1)
    ops.colmax_abs(x2, cm)
    assert torch.equal(cm, torch.maximum(want1, x2.float().abs().amax(dim=0)))
    cm2 = ops.colmax_abs(x2.reshape(1, -1, k))        # leading dims flatten, fresh vector
    assert torch.equal(cm2, x2.float().abs().amax(dim=0))


def test_smooth_ln_fcs_closed_forms():
    _say("smooth_ln_fcs")
    from mindpipe_amd.smoothquant import compute_smooth_scales, smooth_ln_fcs_llama_like
    rng = np.random.default_rng(7)
    k = 512
    w = [(rng.standard_normal((n, k)) * 0.05).astype(np.float16) for n in (384, 128)]
    a = (np.abs(rng.standard_normal(k)) * 6).astype(np.float32)
    lnw = (1 + 0.1 * rng.standard_normal(k)).astype(np.float16)
    fcs = [_lin_from(x, torch.float16) for x in w]
    ln = nn.LayerNorm(k).half().to(DEV)
    with torch.no_grad():
        ln.weight.copy_(torch.from_numpy(lnw))
    s = compute_smooth_scales(fcs, torch.from_numpy(a), 0.5).cpu().numpy()
    smooth_ln_fcs_llama_like(ln, fcs, torch.from_numpy(a), 0.5)
    s32 = s.astype(np.float32)
    assert np.array_equal(ln.weight.detach().cpu().numpy(), (lnw.astype(np.float32) / s32).astype(np.float16))
    for fc, x in zip(fcs, w):
        assert np.array_equal(fc.weight.detach().cpu().numpy(), (x.astype(np.float32) * s32).astype(np.float16))


def _tiny_llama():
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(0)
    cfg = LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, vocab_size=512)
    return LlamaForCausalLM(cfg).half().to(DEV).eval()


def test_get_act_scales_and_smooth_lm_on_tiny_llama():
    _say("get_act_scales / smooth_lm")
    from mindpipe_amd.smoothquant import get_act_scales, smooth_lm
    model = _tiny_llama()
    g = torch.Generator().manual_seed(2)
    batches = [(torch.randint(0, 512, (2, 24), generator=g), None) for _ in range(3)]
    scales = get_act_scales(model, batches)
    # the same statistic with torch hooks
    want = {}

    def hook(_m, inp, _o, name):
        t = inp[0].reshape(-1, inp[0].shape[-1]).abs().amax(dim=0).float().cpu()
        want[name] = torch.maximum(want[name], t) if name in want else t

    hs = [m.register_forward_hook(lambda m_, i_, o_, n=f"model.{n}": hook(m_, i_, o_, n))
          for n, m in model.model.named_modules() if isinstance(m, nn.Linear)]
    with torch.no_grad():
        for ids, _ in batches:
            model(input_ids=ids.to(DEV), use_cache=False)
    for h in hs:
        h.remove()
    assert sorted(scales) == sorted(want) and len(scales) == 14
    for key in want:
        assert torch.equal(scales[key], want[key]), key
    ids = batches[0][0].to(DEV)
    with torch.no_grad():
        before = model(ids).logits.float()
    smooth_lm(model, scales, alpha=0.85)
    with torch.no_grad():
        after = model(ids).logits.float()
    rel = ((after - before).norm() / before.norm()).item()
    assert rel < 1e-2, rel    # the smoothing identity, up to the fp16 roundings of the rescaled weights
